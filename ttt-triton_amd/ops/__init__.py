from ops.ttt_linear import ttt_linear  # noqa: F401
