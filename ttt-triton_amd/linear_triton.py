"""Drop-in for the reference's linear_triton.py: `TritonLinear` with the same
apply() signature and layouts (linear_triton.py:12-60), running the HIP
kernels of libttt_amd.so.  The arithmetic is the ops path's (dual form with a
general KxK eta, LayerNorm eps 1e-8, dense eta gradient); for the row-constant
eta that ttt_layer.py builds it is the function the Triton kernels compute."""

from ttt_amd.linear import TTTLinearFunction


class TritonLinear(TTTLinearFunction):
    # single-GPU build: head sharding through DTensor local_map is not used
    sharded_mode = False


__all__ = ["TritonLinear"]
