"""vertical_and_slash attention on MI355X.

Drop-in for MInference-NPU/minference/ops/vertical_slash_kernel_npu.py:
  vertical_slash_sparse_attention   :518-599
and for the per-head estimator + attention of
MInference-NPU/minference/modules/minference_forward.py:
  _vertical_and_slash_kernel        :140-167
with the visibility of the reference's production mask (_build_vs_mask_direct,
:282-367): query block bq sees the 64-key window below each slash s (ending at
64 (bq + 1) - s) and every vertical column, under the causal mask.  The
library builds a tile list per (head, query block) on the GPU and runs the
same flash kernel as the other patterns; scattered vertical columns are
gathered into dense tiles.  No token mask is formed, so there is no length
cap from mask memory (the reference falls back to causal dense above 16384
tokens, :566-576; this build computes the pattern up to MSA_VS_MAX_SEQ).
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _abi
from .common import (VS_HEAD_DIMS, accepts_float32, check_bnsd, check_supported, kernel_view,
                     make_out, require_kernel_head_dim, sparse_scale)

__all__ = [
    "vertical_slash_sparse_attention",
    "vertical_and_slash_estimate",
    "vertical_and_slash_attention",
    "canonical_vertical_lists",
    "vs_sizes",
]

LAST_Q = 64  # query rows the estimator scores (minference_forward.py:43)


def vs_sizes(s: int, vertical_size: int, slash_size: int):
    """Clamped counts of minference_forward.py:146-147."""
    return min(s, max(int(vertical_size), 30)), min(s, max(int(slash_size), 50))

_DEFAULT_BLOCK_SIZE = 64


def canonical_vertical_lists(v_idx: torch.Tensor, s_k: int):
    """Vertical ids [..., nv] -> (ids, counts): clamped into [0, s_k) as the
    reference does (:346), sorted, repeats dropped (its scatter is a set, :347-351),
    valid ids first.  int32 contiguous."""
    ids = v_idx.long().clamp(0, s_k - 1).sort(dim=-1).values
    nv = ids.shape[-1]
    keep = torch.ones_like(ids, dtype=torch.bool)
    keep[..., 1:] = ids[..., 1:] != ids[..., :-1]
    pos = torch.arange(nv, device=ids.device)
    order = ((~keep).long() * (nv + 1) + pos).argsort(dim=-1)
    ids = ids.gather(-1, order)
    cnt = keep.sum(dim=-1)
    ids = torch.where(pos < cnt[..., None], ids, torch.zeros_like(ids))
    return ids.to(torch.int32).contiguous(), cnt.to(torch.int32).contiguous()


def _check_vs_shape(q: torch.Tensor, k: torch.Tensor) -> None:
    assert q.shape[2] == k.shape[2], (
        "vertical_and_slash needs S_q == S_k (full prefill); got "
        f"S_q={q.shape[2]}, S_k={k.shape[2]}"
    )
    if q.shape[2] > _abi.MSA_VS_MAX_SEQ:
        raise NotImplementedError(
            f"vertical_and_slash supports S <= {_abi.MSA_VS_MAX_SEQ} on MI355X, got {q.shape[2]}"
        )


@accepts_float32(("q", "k"), has_out=False)
def vertical_and_slash_estimate(q: torch.Tensor, k: torch.Tensor, vertical_size: int,
                                slash_size: int):
    """Vertical and slash indices of every head (minference_forward.py:140-165):
    ``(v_idx [B,H,nv] ascending, s_idx [B,H,ns] descending)`` int64, with
    nv, ns from :func:`vs_sizes`.  k may have fewer heads (GQA)."""
    assert q.dim() == 4 and k.dim() == 4
    check_supported(q, k)
    require_kernel_head_dim(q.shape[-1], "vertical_and_slash", VS_HEAD_DIMS)
    _check_vs_shape(q, k)
    q, k = kernel_view(q), kernel_view(k)
    B, H, S, _ = q.shape
    nv, ns = vs_sizes(S, vertical_size, slash_size)
    v_idx = torch.empty((B, H, nv), dtype=torch.int32, device=q.device)
    s_idx = torch.empty((B, H, ns), dtype=torch.int32, device=q.device)
    v_cnt = torch.empty((B, H), dtype=torch.int32, device=q.device)
    s_cnt = torch.empty((B, H), dtype=torch.int32, device=q.device)
    step = _abi.MSA_MAX_HEADS
    for h0 in range(0, H, step):
        h1 = min(H, h0 + step)
        n = h1 - h0
        vi = torch.empty((B, n, nv), dtype=torch.int32, device=q.device)
        si = torch.empty((B, n, ns), dtype=torch.int32, device=q.device)
        vc = torch.empty((B, n), dtype=torch.int32, device=q.device)
        sc = torch.empty((B, n), dtype=torch.int32, device=q.device)
        _abi.vs_estimate(q, k, list(range(h0, h1)), [nv] * n, [ns] * n, vi, vc, si, sc)
        v_idx[:, h0:h1], s_idx[:, h0:h1] = vi, si
        v_cnt[:, h0:h1], s_cnt[:, h0:h1] = vc, sc
    return v_idx.long(), s_idx.long()


@accepts_float32(("q", "k", "v"))
def vertical_and_slash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                 vertical_size: int, slash_size: int, *,
                                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Estimator + vertical-slash attention for every head, the reference's
    _vertical_and_slash_kernel (minference_forward.py:140-167) on
    ``[B, H, S, D]`` tensors (k, v with H heads)."""
    check_bnsd(q, k, v)
    check_supported(q, k, v)
    require_kernel_head_dim(q.shape[-1], "vertical_and_slash", VS_HEAD_DIMS)
    _check_vs_shape(q, k)
    q, k, v = kernel_view(q), kernel_view(k), kernel_view(v)
    v_idx, s_idx = vertical_and_slash_estimate(q, k, vertical_size, slash_size)
    v_ids = v_idx.to(torch.int32).contiguous()
    v_cnt = torch.full(v_ids.shape[:2], v_ids.shape[-1], dtype=torch.int32, device=q.device)
    result = make_out(q, out)
    return run_vs_heads(q, k, v, result, v_ids, v_cnt, s_idx.to(torch.int32).contiguous(),
                        sparse_scale(q.shape[-1]))


def _vs_head_chunks(batch: int, n_heads: int):
    """Head ranges with batch * heads <= MSA_MAX_HEADS per library call."""
    step = max(1, _abi.MSA_MAX_HEADS // max(batch, 1))
    for h0 in range(0, n_heads, step):
        yield h0, min(n_heads, h0 + step)


def run_vs_heads(q, k, v, result, v_ids, v_cnt, s_idx, scale):
    """All heads of q as vertical_and_slash heads (slot h = head h); lists
    [B, H, n] int32 contiguous on q's device."""
    B, H = q.shape[0], q.shape[1]
    if B > _abi.MSA_MAX_HEADS:
        raise ValueError(f"vertical_and_slash supports batch <= {_abi.MSA_MAX_HEADS}")
    s_cnt = torch.full((B, H), s_idx.shape[-1], dtype=torch.int32, device=q.device)
    for h0, h1 in _vs_head_chunks(B, H):
        n = h1 - h0
        heads = [(_abi.MSA_KIND_VS, v_ids.shape[-1], s_idx.shape[-1], s, scale) for s in range(n)]
        lists = (v_ids[:, h0:h1].contiguous(), v_cnt[:, h0:h1].contiguous(),
                 s_idx[:, h0:h1].contiguous(), s_cnt[:, h0:h1].contiguous())
        _abi.layer_attention(q[:, h0:h1], k[:, h0:h1], v[:, h0:h1], result[:, h0:h1], heads,
                             vs=lists)
    return result


@accepts_float32(("query", "key", "value"))
def vertical_slash_sparse_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    v_idx: torch.Tensor,
    s_idx: torch.Tensor,
    block_size_M: int = _DEFAULT_BLOCK_SIZE,
    block_size_N: int = _DEFAULT_BLOCK_SIZE,
    *,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Vertical-slash causal attention.

    Args:
        query, key, value: ``[B, H, S, D]`` (BNSD), RoPE applied, ``repeat_kv``-ed.
        v_idx: ``[B, H, NNZ_V]`` vertical column ids (any order; clamped to
               ``[0, S)``, repeats count once).
        s_idx: ``[B, H, NNZ_S]`` slash offsets ``s`` (the diagonal ``j = i - s``).
        block_size_M, block_size_N: must be 64.
        out: optional output (query's dtype or float32).

    Returns ``[B, H, S, D]`` in query's dtype (or ``out``).  The softmax scale
    is ``(padded D) ** -0.5`` (the reference pads D to 16/32/64/128/256/512
    first, :581-587).
    """
    assert query.dim() == 4, f"query must be 4-D [B,H,S,D], got {query.dim()}-D"
    _check_vs_shape(query, key)
    assert block_size_M == _DEFAULT_BLOCK_SIZE and block_size_N == _DEFAULT_BLOCK_SIZE, (
        f"block sizes must be {_DEFAULT_BLOCK_SIZE}, got {block_size_M}/{block_size_N}"
    )
    check_bnsd(query, key, value)
    check_supported(query, key, value)
    require_kernel_head_dim(query.shape[-1], "vertical_and_slash", VS_HEAD_DIMS)
    B, H, S, _ = query.shape
    if tuple(v_idx.shape[:2]) != (B, H) or tuple(s_idx.shape[:2]) != (B, H):
        raise ValueError("v_idx / s_idx must be [B, H, n] for q of shape " f"{tuple(query.shape)}")
    q, k, v = kernel_view(query), kernel_view(key), kernel_view(value)
    v_ids, v_cnt = canonical_vertical_lists(v_idx.to(q.device), S)
    s = s_idx.to(device=q.device, dtype=torch.int32).contiguous()
    result = make_out(q, out)
    return run_vs_heads(q, k, v, result, v_ids, v_cnt, s, sparse_scale(q.shape[-1]))
