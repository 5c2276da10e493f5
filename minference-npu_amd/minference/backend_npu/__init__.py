"""Import-path alias of ``minference.backend`` for code written against the
reference's ``minference.backend_npu`` (backend_npu/__init__.py)."""

from ..backend.attention import decode_dense, dense_attention, prefill_dense

__all__ = ["dense_attention", "prefill_dense", "decode_dense"]
