"""Dense attention on MI355X.

Drop-in for ``dense_attention`` / ``prefill_dense`` / ``decode_dense`` of
MInference-NPU/minference/backend_npu/attention.py:192-314.  Prefill runs the
same tile-list kernel as the sparse kinds with every causal tile listed;
decode (one query row) runs a split-K kernel that reads the cache in place.
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _abi
from ..ops.common import (accepts_float32, check_bnsd, check_supported, dense_scale, head_chunks,
                          padded_call)

__all__ = ["dense_attention", "prefill_dense", "decode_dense"]


@accepts_float32(("q", "k", "v"))
def dense_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    scale: Optional[float] = None,
    causal: bool = True,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Dense attention, ``[B, H, S, D]`` in and out.

    causal=True: query i sees key j iff j <= i + (S_k - S_q) (S_q <= S_k).
    causal=False: every query sees every key, any S_q and S_k (reference
    :221-230).  ``scale`` defaults to 1/sqrt(D) of the unpadded head_dim
    (reference :210-211).
    """
    check_bnsd(q, k, v)
    check_supported(q, k, v, allow_longer_q=not causal)
    s = dense_scale(q.shape[-1]) if scale is None else float(scale)
    kind = _abi.MSA_KIND_DENSE if causal else _abi.MSA_KIND_FULL

    def run(q, k, v, result):
        for h0, h1 in head_chunks(q.shape[1]):
            heads = [(kind, 0, 0, -1, s)] * (h1 - h0)
            _abi.layer_attention(q[:, h0:h1], k[:, h0:h1], v[:, h0:h1], result[:, h0:h1], heads)

    return padded_call(q, k, v, out, run)


def prefill_dense(q, k, v, *, scale: Optional[float] = None, causal: bool = True):
    """Same as dense_attention (reference :258-271)."""
    return dense_attention(q, k, v, scale=scale, causal=causal)


@accepts_float32(("q", "k_cache", "v_cache"))
def decode_dense(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    *,
    scale: Optional[float] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """One query row per head against the whole cache (reference :274-314).

    q ``[B, H, 1, D]``; k_cache / v_cache ``[B, H_kv, S_kv, D]`` with
    ``H % H_kv == 0`` (the reference passes ``H_kv == H``); every key is
    visible; ``scale`` defaults to 1/sqrt(D).  Returns ``[B, H, 1, D]`` in q's
    dtype (or writes ``out``, q's dtype or fp32).
    """
    assert q.dim() == 4 and k_cache.dim() == 4, "q and the caches must be 4-D [B,H,S,D]"
    assert v_cache.shape == k_cache.shape, (
        f"v_cache shape {tuple(v_cache.shape)} != k_cache shape {tuple(k_cache.shape)}")
    assert q.shape[0] == k_cache.shape[0] and q.shape[-1] == k_cache.shape[-1], (
        f"q/k_cache B/D mismatch; q={tuple(q.shape)} k={tuple(k_cache.shape)}")
    if q.shape[1] % k_cache.shape[1] != 0:
        raise ValueError(f"q heads {q.shape[1]} not a multiple of cache heads {k_cache.shape[1]}")
    if q.shape[2] != 1:
        raise NotImplementedError("decode_dense takes one query row; use dense_attention for "
                                  "q_len > 1")
    check_supported(q, k_cache, v_cache)
    s = dense_scale(q.shape[-1]) if scale is None else float(scale)
    return padded_call(q, k_cache, v_cache, out,
                       lambda q, k, v, r: _abi.decode_attention(q, k, v, r, s))
