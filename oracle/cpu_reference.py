"""torch-CPU fp32 restatement of the reference's CPU attention paths, for
timing the reference's own CPU algorithm on the host (the benchmark's
``cpu_baseline``).

TEST INFRASTRUCTURE ONLY: used by bench.py's CPU baseline leg and by
tests/test_cpu_reference.py, never by the product package.

The reference runs these ops on the CPU when no NPU is present; this file
performs the same torch operations in the same order, so its timing is the
reference CPU path's timing:
  stream_llm  : streaming_forward (minference/ops/streaming_kernel_npu.py:
                349-397) pads D to the next allowed size (96 -> 128, :377-381)
                and calls _streaming_pytorch_ref (:94-146): per query chunk of
                max(64, min(S_q, 4M // S_k)) rows, fp32 logits against every
                key, sink/band/causal mask, softmax, nan_to_num, PV.
  block_sparse: block_sparse_attention (minference/ops/block_sparse_kernel_npu.py:
                609-709) pads D the same way and, off the NPU, calls
                _block_sparse_pytorch_ref (:325-348): the selector (:230-263),
                the token mask (:266-317), then fp32 masked softmax over all
                S_q x S_k logits and PV.  As written it holds [B, H, S, S] fp32
                logits (34 GB for 32 heads at S = 16384); here it runs one head
                at a time, the same operations per head.
Parity of these functions with the numpy oracle is checked in
tests/test_cpu_reference.py.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

ALLOWED_HEAD_DIMS = (16, 32, 64, 128, 256, 512)


def _padded(x: torch.Tensor) -> torch.Tensor:
    """Zero pad D to the next allowed head size (streaming_kernel_npu.py:377-381,
    block_sparse_kernel_npu.py:651-656)."""
    d = x.shape[-1]
    target = next(c for c in ALLOWED_HEAD_DIMS if c >= d)
    return F.pad(x, (0, target - d)) if target != d else x


def streaming_reference(q, k, v, n_init: int, n_local: int) -> torch.Tensor:
    """stream_llm on the CPU as the reference runs it (D padded, chunked
    full-row fp32 logits, masked softmax); returns [B, H, S_q, D] in q's dtype."""
    d0 = q.shape[-1]
    q, k, v = _padded(q), _padded(k), _padded(v)
    _, _, s_q, d = q.shape
    s_k = k.shape[2]
    scale = 1.0 / math.sqrt(d)
    rows = max(64, min(s_q, (4 * 1024 * 1024) // max(1, s_k)))
    keys = torch.arange(s_k)
    kt = k.float().transpose(-2, -1)
    vf = v.float()
    out = torch.empty_like(q)
    for c0 in range(0, s_q, rows):
        c1 = min(c0 + rows, s_q)
        pos = torch.arange(s_k - s_q + c0, s_k - s_q + c1)[:, None]
        seen = (keys[None, :] <= pos) & ((keys[None, :] > pos - n_local) | (keys[None, :] < n_init))
        logits = torch.matmul(q[:, :, c0:c1].float(), kt) * scale
        logits = logits.masked_fill(~seen, float("-inf"))
        probs = torch.nan_to_num(torch.softmax(logits, dim=-1), nan=0.0)
        out[:, :, c0:c1] = torch.matmul(probs, vf).to(q.dtype)
    return out[..., :d0]


def select_blocks(q, k, topk: int, block: int = 64) -> torch.Tensor:
    """The reference selector's torch steps (block_sparse_kernel_npu.py:240-263):
    pooling in the input dtype, fp32 scores times D**-0.5 (padded D), block-causal
    -inf mask, topk, sort."""
    b, h, s_q, d = q.shape
    s_k = k.shape[2]
    pq, pk = (-s_q) % block, (-s_k) % block
    qp = F.pad(q, (0, 0, 0, pq)) if pq else q
    kp = F.pad(k, (0, 0, 0, pk)) if pk else k
    n_bq, n_bk = qp.shape[2] // block, kp.shape[2] // block
    q_pool = qp.reshape(b, h, n_bq, block, d).mean(dim=3).to(torch.float32)
    k_pool = kp.reshape(b, h, n_bk, block, d).mean(dim=3).to(torch.float32)
    scores = torch.matmul(q_pool, k_pool.transpose(-2, -1)) * (d ** -0.5)
    allowed = torch.arange(n_bq)[:, None] >= torch.arange(n_bk)[None, :]
    scores.masked_fill_(~allowed, float("-inf"))
    return torch.topk(scores, min(topk, n_bk), dim=-1).indices.sort(dim=-1).values


def block_sparse_reference(q, k, v, topk: int, block: int = 64) -> torch.Tensor:
    """block_sparse on the CPU as the reference runs it, one head at a time:
    selector, token mask (selected blocks and token causality), fp32 masked
    softmax over all logits, PV; returns [B, H, S_q, D] in q's dtype."""
    d0 = q.shape[-1]
    q, k, v = _padded(q), _padded(k), _padded(v)
    b, h, s_q, d = q.shape
    s_k = k.shape[2]
    scale = d ** -0.5
    out = torch.empty_like(q)
    causal = torch.arange(s_k - s_q, s_k)[:, None] >= torch.arange(s_k)[None, :]
    n_bq, n_bk = -(-s_q // block), -(-s_k // block)
    for hh in range(h):
        sl = slice(hh, hh + 1)
        ids = select_blocks(q[:, sl], k[:, sl], topk, block)
        chosen = torch.zeros(b, 1, n_bq, n_bk, dtype=torch.bool)
        chosen.scatter_(-1, ids, True)
        tok = chosen.repeat_interleave(block, dim=2).repeat_interleave(block, dim=3)
        seen = tok[:, :, :s_q, :s_k] & causal
        logits = torch.matmul(q[:, sl].float(), k[:, sl].float().transpose(-2, -1)) * scale
        logits.masked_fill_(~seen, float("-inf"))
        probs = torch.nan_to_num(torch.softmax(logits, dim=-1), nan=0.0)
        out[:, sl] = torch.matmul(probs, v[:, sl].float()).to(q.dtype)
    return out[..., :d0]
