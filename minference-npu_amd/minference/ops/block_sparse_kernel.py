"""block_sparse attention on MI355X: GPU block top-k estimator + gather-free
block-sparse flash kernel.

Drop-in for MInference-NPU/minference/ops/block_sparse_kernel_npu.py:
  block_sparse_attention                 :609-709
  _select_block_sparse_topk_indices      :230-263
  _block_sparse_tilelang_npu_with_indices :452-601 (fixed-index kernel call)
The kernel walks each (head, 64-row query block)'s id list directly; there is
no fold of heads into the batch, no token-index expansion and no padding of
small head counts.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from .. import _abi
from .common import (accepts_float32, check_bnsd, check_supported, head_chunks, kernel_head_dim,
                     kernel_view, pad_head_dim, padded_call, sparse_scale)

__all__ = [
    "block_sparse_attention",
    "select_block_sparse_topk_indices",
    "block_sparse_attention_with_indices",
]

_DEFAULT_BLOCK_SIZE = 64


# Block sizes of the selector and the token mask: the attention kernels walk
# 64-token tiles, so a block of 64 m tokens is m consecutive tiles.
def _check_block_size(block_size: int) -> None:
    bs = int(block_size)
    if bs < _abi.MSA_BLOCK or bs % _abi.MSA_BLOCK:
        raise NotImplementedError(
            f"block_size={block_size}: the MI355X kernels take multiples of {_abi.MSA_BLOCK}"
        )


def select_flags(force_first: bool = False, force_diag: bool = False) -> int:
    """Selector flags: block 0 / the query block's own block always kept,
    inside the top-k (an option of this build; the reference selector has
    none)."""
    return ((_abi.MSA_SELECT_FORCE_FIRST if force_first else 0)
            | (_abi.MSA_SELECT_FORCE_DIAG if force_diag else 0))


def _estimate(q: torch.Tensor, k: torch.Tensor, topk: int, scale: float, flags: int = 0,
              block: int = _DEFAULT_BLOCK_SIZE):
    """Run the estimator for every head of q (kernel views at the kernel
    head dim; ``scale`` from the original head_dim) with blocks of ``block``
    tokens.

    Returns a list of (h0, h1, idx, cnt) per head chunk of at most
    MSA_MAX_HEADS heads, idx/cnt int32 contiguous [B, h1-h0, n_qb(, topk)].
    """
    B, H, S_q, _ = q.shape
    n_qb = math.ceil(S_q / block)
    chunks = []
    for h0, h1 in head_chunks(H):
        n = h1 - h0
        idx = torch.empty((B, n, n_qb, topk), dtype=torch.int32, device=q.device)
        cnt = torch.empty((B, n, n_qb), dtype=torch.int32, device=q.device)
        _abi.block_estimate(
            q[:, h0:h1], k[:, h0:h1], list(range(n)), [topk] * n, topk, scale, idx, cnt,
            flags=flags, block=block,
        )
        chunks.append((h0, h1, idx, cnt))
    return chunks


@accepts_float32(("q", "k"), has_out=False)
def select_block_sparse_topk_indices(
    q: torch.Tensor,
    k: torch.Tensor,
    topk_blocks: int,
    block_size: int = _DEFAULT_BLOCK_SIZE,
    *,
    return_counts: bool = False,
    force_first: bool = False,
    force_diag: bool = False,
):
    """Selected K-block ids per query block, ``[B, H, n_q_blocks, topk]`` int64.

    Same pooling, scale and block-causal rule as the reference selector
    (:230-263).  The first ``min(topk, bq+1)`` ids of each row are the chosen
    causal blocks ascending (ties -> lower id).  The remaining slots (rows
    with fewer causal blocks than ``topk``) hold the next future ids; the
    reference fills them with ``torch.topk``'s choice among ``-inf`` scores,
    and the token-level causal mask discards them in both implementations.
    With ``return_counts=True`` also returns the per-row counts of leading ids
    some row of the query block attends: min(topk, bq+1), plus, when
    S_q < S_k, the surplus ids that lie before the block's last absolute row.
    ``force_first`` / ``force_diag`` (not in the reference) keep block 0 /
    the query block's own block in every row, inside the top-k.
    """
    check_bnsd(q, k)
    check_supported(q, k)
    _check_block_size(block_size)
    scale = sparse_scale(q.shape[-1])
    dk = kernel_head_dim(q.shape[-1])
    q, k = kernel_view(pad_head_dim(q, dk)), kernel_view(pad_head_dim(k, dk))
    bs = int(block_size)
    n_kb = math.ceil(k.shape[2] / bs)
    topk = min(max(1, int(topk_blocks)), n_kb)
    chunks = _estimate(q, k, topk, scale, select_flags(force_first, force_diag), bs)
    idx = torch.cat([c[2] for c in chunks], dim=1).long()
    if return_counts:
        return idx, torch.cat([c[3] for c in chunks], dim=1).long()
    return idx


# reference-private name kept for drop-in callers and tests
_select_block_sparse_topk_indices = select_block_sparse_topk_indices


@accepts_float32(("q", "k", "v"))
def block_sparse_attention_with_indices(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    block_indices: torch.Tensor,
    block_size: int = _DEFAULT_BLOCK_SIZE,
    *,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Block-sparse attention for a fixed ``[B, H, n_q_blocks, topk]`` id tensor
    (the kernel call of :452-601, minus its fp16-only and fold-into-batch
    restrictions).  Ids outside [0, n_k_blocks) are ignored; duplicated ids
    count once; future blocks are removed by the token causal mask."""
    check_bnsd(q, k, v)
    check_supported(q, k, v)
    _check_block_size(block_size)
    B, H, S_q, _ = q.shape
    bs = int(block_size)
    if tuple(block_indices.shape[:3]) != (B, H, math.ceil(S_q / bs)):
        raise ValueError(
            "block_indices shape must be [B,H,n_q_blocks,topk_blocks]; "
            f"got {tuple(block_indices.shape)} for q={tuple(q.shape)} block_size={block_size}"
        )
    ids = block_indices.to(q.device)
    if bs != _abi.MSA_BLOCK:
        ids = tile_ids(ids, bs, math.ceil(S_q / _abi.MSA_BLOCK))
    n_kb = math.ceil(k.shape[2] / _abi.MSA_BLOCK)
    idx, cnt = canonical_block_lists(ids, n_kb)
    topk = idx.shape[-1]
    chunks = []
    for h0, h1 in head_chunks(H):
        chunks.append((h0, h1, idx[:, h0:h1].contiguous(), cnt[:, h0:h1].contiguous()))
    scale = sparse_scale(q.shape[-1])
    return padded_call(q, k, v, out, lambda q, k, v, r: _run(q, k, v, chunks, topk, scale, r))


def tile_ids(block_indices: torch.Tensor, block_size: int, n_qb: int) -> torch.Tensor:
    """Ids of ``block_size``-token blocks [B, H, n_q_blocks, topk] as ids of
    the kernels' 64-token tiles [B, H, n_qb, topk * m] (m = block_size / 64):
    block J is tiles m J .. m J + m - 1, and 64-row query block bq takes the
    list of its block bq // m.  The token visibility is unchanged: a key is
    in a selected block iff its tile is among that block's tiles.  Ids
    outside the key range stay outside it (negative ones stay negative)."""
    m = int(block_size) // _abi.MSA_BLOCK
    ids = block_indices.long()
    tiles = (ids.unsqueeze(-1) * m + torch.arange(m, device=ids.device)).flatten(-2)
    rows = torch.arange(n_qb, device=ids.device) // m
    return tiles[:, :, rows]


def canonical_block_lists(block_indices: torch.Tensor, n_kb: int):
    """Turn arbitrary per-row block ids into the kernel's list format: the
    distinct ids in [0, n_kb) ascending first, ``cnt`` = how many.  This is the
    set semantics of the reference's scatter into a block mask
    (block_sparse_kernel_npu.py:290-291): repeats count once and ids outside
    the key range select nothing.  Returns int32 (idx, cnt)."""
    ids = block_indices.long()
    topk = ids.shape[-1]
    valid = (ids >= 0) & (ids < n_kb)
    ids = torch.where(valid, ids, torch.full_like(ids, n_kb)).sort(dim=-1).values
    keep = ids < n_kb
    keep[..., 1:] &= ids[..., 1:] != ids[..., :-1]
    pos = torch.arange(topk, device=ids.device)
    order = ((~keep).long() * (topk + 1) + pos).argsort(dim=-1)
    ids = ids.gather(-1, order)
    cnt = keep.sum(dim=-1)
    ids = torch.where(pos < cnt[..., None], ids, torch.zeros_like(ids))
    return ids.to(torch.int32).contiguous(), cnt.to(torch.int32).contiguous()


def _run(q, k, v, chunks, topk, scale, result):
    for h0, h1, idx, cnt in chunks:
        n = h1 - h0
        heads = [(_abi.MSA_KIND_BLOCK, topk, 0, s, scale) for s in range(n)]
        _abi.layer_attention(
            q[:, h0:h1], k[:, h0:h1], v[:, h0:h1], result[:, h0:h1], heads,
            idx=idx, cnt=cnt, idx_slots=n, topk_max=topk,
        )
    return result


@accepts_float32(("q", "k", "v"))
def block_sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    topk_blocks: int,
    block_size: int = _DEFAULT_BLOCK_SIZE,
    *,
    out: Optional[torch.Tensor] = None,
    force_first: bool = False,
    force_diag: bool = False,
) -> torch.Tensor:
    """Block-sparse causal attention.

    Args:
        q, k, v:     ``[B, H, S, D]`` (BNSD), RoPE applied, ``repeat_kv``-ed.
        topk_blocks: K blocks kept per query block (clamped to >= 1 and to the
                     number of K blocks, as in the reference).
        block_size:  a multiple of 64 tokens (the attention kernels walk
                     64-token tiles; a larger block is its consecutive tiles).
        out:         optional output (q's dtype or float32).
        force_first, force_diag: keep block 0 / the diagonal block in every
                     selection (options of this build, off by default: the
                     reference's selector is the plain top-k).

    Returns ``[B, H, S, D]`` in q's dtype (or ``out``).
    """
    check_bnsd(q, k, v)
    check_supported(q, k, v)
    _check_block_size(block_size)
    if int(block_size) != _abi.MSA_BLOCK:
        ids = select_block_sparse_topk_indices(q, k, topk_blocks, block_size,
                                               force_first=force_first, force_diag=force_diag)
        return block_sparse_attention_with_indices(q, k, v, ids, block_size, out=out)
    n_kb = math.ceil(k.shape[2] / _abi.MSA_BLOCK)
    topk = min(max(1, int(topk_blocks)), n_kb)
    scale = sparse_scale(q.shape[-1])
    flags = select_flags(force_first, force_diag)

    def run(q, k, v, result):
        _run(q, k, v, _estimate(q, k, topk, scale, flags), topk, scale, result)

    return padded_call(q, k, v, out, run)
