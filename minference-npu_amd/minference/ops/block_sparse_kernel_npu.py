"""Import-path alias of ``minference.ops.block_sparse_kernel`` for code written
against the reference module name (ops/block_sparse_kernel_npu.py)."""

from .block_sparse_kernel import (
    _select_block_sparse_topk_indices,
    block_sparse_attention,
    block_sparse_attention_with_indices,
    select_block_sparse_topk_indices,
)

__all__ = ["block_sparse_attention"]
