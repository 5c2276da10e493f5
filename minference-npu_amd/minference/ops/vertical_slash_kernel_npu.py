"""Import-path alias of ``minference.ops.vertical_slash_kernel`` for code
written against the reference module name (ops/vertical_slash_kernel_npu.py)."""

from .vertical_slash_kernel import vertical_slash_sparse_attention

__all__ = ["vertical_slash_sparse_attention"]
