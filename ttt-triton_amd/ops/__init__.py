from ops.ttt_linear import ttt_linear  # noqa: F401
from ops.ttt_mlp import ttt_mlp  # noqa: F401
