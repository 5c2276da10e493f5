"""Sparse prefill attention ops (HIP kernels behind the C ABI in include/msa.h)."""
