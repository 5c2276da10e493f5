"""Import-path alias: ``minference.backend_npu.attention`` -> ``minference.backend.attention``."""

from ..backend.attention import dense_attention, prefill_dense

__all__ = ["dense_attention", "prefill_dense"]
