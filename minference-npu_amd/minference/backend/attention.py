"""Dense causal attention on MI355X.

Drop-in for ``dense_attention`` / ``prefill_dense`` of
MInference-NPU/minference/backend_npu/attention.py:192-271.  It runs the same
tile-list kernel as the sparse kinds with every causal tile listed.
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _abi
from ..ops.common import check_bnsd, check_supported, dense_scale, head_chunks, kernel_view, make_out

__all__ = ["dense_attention", "prefill_dense"]


def dense_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    scale: Optional[float] = None,
    causal: bool = True,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Dense causal attention, ``[B, H, S, D]`` in and out.

    Query i sees key j iff j <= i + (S_k - S_q).  ``scale`` defaults to
    1/sqrt(D) of the unpadded head_dim (reference :210-211).  Only the causal
    prefill form is implemented (``causal=False`` belongs to decode, which is
    outside this build).
    """
    if not causal:
        raise NotImplementedError("dense_attention(causal=False) is not part of the MI355X prefill path")
    check_bnsd(q, k, v)
    check_supported(q, k, v)
    q, k, v = kernel_view(q), kernel_view(k), kernel_view(v)
    result = make_out(q, out)
    s = dense_scale(q.shape[-1]) if scale is None else float(scale)
    for h0, h1 in head_chunks(q.shape[1]):
        heads = [(_abi.MSA_KIND_DENSE, 0, 0, -1, s)] * (h1 - h0)
        _abi.layer_attention(q[:, h0:h1], k[:, h0:h1], v[:, h0:h1], result[:, h0:h1], heads)
    return result


def prefill_dense(q, k, v, *, scale: Optional[float] = None, causal: bool = True):
    """Same as dense_attention (reference :258-271)."""
    return dense_attention(q, k, v, scale=scale, causal=causal)
