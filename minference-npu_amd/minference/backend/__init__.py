"""Dense attention on MI355X (the dense-others head kind and the dense baseline)."""

from .attention import dense_attention, prefill_dense

__all__ = ["dense_attention", "prefill_dense"]
