"""stream_llm (attention sinks + causal local band) on MI355X.

Drop-in for ``streaming_forward`` of
MInference-NPU/minference/ops/streaming_kernel_npu.py:349-397.  One fused HIP
launch covers the sink columns and the band (the reference runs a band FA, a
sink FA and an fp32 LSE merge, :233-341); the online softmax inside the kernel
is that merge.
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _abi
from .common import (accepts_float32, check_bnsd, check_supported, head_chunks, padded_call,
                     sparse_scale)

__all__ = ["streaming_forward"]


@accepts_float32(("q", "k", "v"))
def streaming_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    n_init: int,
    n_local: int,
    *,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Sink + sliding-window attention (A-shape / streaming-LLM).

    Args:
        q, k, v: ``[B, H, S, D]`` (BNSD), RoPE applied, K/V already
                 ``repeat_kv``-ed or with ``H % H_kv == 0`` heads.
        n_init:  number of sink tokens (always visible); <= 0 means none.
        n_local: width of the causal sliding window.
        out:     optional output (q's dtype or float32), written in place.

    Query i (absolute position a = S_k - S_q + i) sees key j iff
    j <= a and (j > a - n_local or j < n_init).  When S_k <= n_local this is
    causal dense attention, which is the reference's short circuit (:385-390).
    The softmax scale is (padded head_dim)**-0.5 as in the reference; a
    head_dim the kernels are not built for runs zero-padded to the next one.
    """
    check_bnsd(q, k, v)
    check_supported(q, k, v)
    scale = sparse_scale(q.shape[-1])

    def run(q, k, v, result):
        for h0, h1 in head_chunks(q.shape[1]):
            heads = [(_abi.MSA_KIND_STREAM, int(n_init), int(n_local), -1, scale)] * (h1 - h0)
            _abi.layer_attention(
                q[:, h0:h1], k[:, h0:h1], v[:, h0:h1], result[:, h0:h1], heads
            )

    return padded_call(q, k, v, out, run)
