"""Drop-in for kernels/mlp_cached_readout.py: `mlp_cached_readout_triton(XQ_seg,
W1, b1, W2, b2, ln_w, ln_b)` (kernels/mlp_cached_readout.py:112-143), the
fixed-weight TTT-MLP readout XQ_seg + LN_{1e-6}(gelu(XQ_seg W1 + b1) W2 + b2)
returned in float32, as ttt_layer.py:542-552 calls it per cached memo slice.

Each (b,h) chain uses its own weights (the reference kernel's stores all land
on chain 0, so its result is only defined for B*H == 1).  A slice
`W1_memo[:, :, j]` of the forward's memo output is read in place, without the
copy a contiguous layout would need."""

from ttt_amd.mlp import mlp_cached_readout


def mlp_cached_readout_triton(XQ_seg, W1, b1, W2, b2, ln_w, ln_b):
    return mlp_cached_readout(XQ_seg, W1, b1, W2, b2, ln_w, ln_b)


__all__ = ["mlp_cached_readout_triton"]
