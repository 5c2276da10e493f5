"""Dense attention on MI355X (the dense-others head kind and the dense baseline)."""

from .attention import decode_dense, dense_attention, prefill_dense

__all__ = ["dense_attention", "prefill_dense", "decode_dense"]
