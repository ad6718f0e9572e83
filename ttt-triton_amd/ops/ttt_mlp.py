"""Drop-in for ops/ttt_mlp.py: `ttt_mlp(XK, XQ, XV, eta, ln_w, ln_b, W1_init,
b1_init, W2_init, b2_init, checkpoint_group_size) -> [B,NC,K,H,F]`
(ops/ttt_mlp.py:70-99), forward and backward on the HIP kernels.
checkpoint_group_size only sets how often the forward keeps fast-weight
checkpoints for the backward's recompute (<= 0 means one group); results do
not depend on it."""

from ttt_amd.mlp import TTTMLPFunction


def ttt_mlp(XK, XQ, XV, eta, ttt_norm_weight, ttt_norm_bias, W1_init, b1_init, W2_init, b2_init,
            checkpoint_group_size):
    NC = XQ.shape[2]
    G = NC if checkpoint_group_size <= 0 else min(int(checkpoint_group_size), NC)
    out = TTTMLPFunction.apply(ttt_norm_weight, ttt_norm_bias, W1_init, b1_init, W2_init, b2_init,
                               XQ, XV, XK, eta, G, 0)[0]
    return out.permute(0, 2, 3, 1, 4)
