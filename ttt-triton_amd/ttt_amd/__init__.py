"""MI355X (gfx950) TTT-Linear / TTT-MLP inner loop: PyTorch host code over
hand-written HIP kernels behind the C ABI in include/ttt_amd.h."""

from . import _lib  # noqa: F401
from .linear import linear_backward, linear_forward, TTTLinearFunction  # noqa: F401
from .mlp import mlp_backward, mlp_cached_readout, mlp_forward, TTTMLPFunction  # noqa: F401
from .memo import MemoCombineFunction, mlp_memo_combine  # noqa: F401
