"""Drop-in for the reference's mlp_triton.py: `TritonMLP` with the same
apply() signature, layouts and outputs (mlp_triton.py:12-69): (XQW, W1_memo,
b1_memo, W2_memo, b2_memo), memo fp32 and non-differentiable, running the HIP
kernels of libttt_amd.so.  The arithmetic is the ops path's (dual form with a
general KxK eta, LayerNorm eps 1e-8, dense eta gradient)."""

from ttt_amd.mlp import TTTMLPFunction


class TritonMLP(TTTMLPFunction):
    # single-GPU build: head sharding through DTensor local_map is not used
    sharded_mode = False


__all__ = ["TritonMLP"]
