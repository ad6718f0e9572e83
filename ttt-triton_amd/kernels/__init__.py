"""HIP-backed stand-ins for the reference's kernels/ package entry points."""
