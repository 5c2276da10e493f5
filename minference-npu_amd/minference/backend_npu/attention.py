"""Import-path alias: ``minference.backend_npu.attention`` -> ``minference.backend.attention``."""

from ..backend.attention import decode_dense, dense_attention, prefill_dense

__all__ = ["dense_attention", "prefill_dense", "decode_dense"]
