"""Drop-in for ops/ttt_linear.py: `ttt_linear(XK, XQ, XV, eta, ln_w, ln_b,
W1_init, b1_init, checkpoint_group_size) -> [B,NC,K,H,F]` (ops/ttt_linear.py:57-84),
forward and backward on the HIP kernels.  checkpoint_group_size only sets how
often the forward keeps fast-weight checkpoints for the backward's recompute
(<= 0 means one group); results do not depend on it."""

from ttt_amd.linear import TTTLinearFunction


def ttt_linear(XK, XQ, XV, eta, ttt_norm_weight, ttt_norm_bias, W1_init, b1_init, checkpoint_group_size):
    NC = XQ.shape[2]
    G = NC if checkpoint_group_size <= 0 else min(int(checkpoint_group_size), NC)
    out = TTTLinearFunction.apply(ttt_norm_weight, ttt_norm_bias, W1_init, b1_init, XQ, XV, XK, eta, G)
    return out.permute(0, 2, 3, 1, 4)
