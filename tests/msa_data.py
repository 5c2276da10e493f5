"""Synthetic Phi-3-shaped inputs shared by the tests and the benchmark."""

from __future__ import annotations

import numpy as np
import torch


def rope(x: torch.Tensor, theta: float = 10000.0, offset: int = 0) -> torch.Tensor:
    """HF rotate_half RoPE on [B, H, S, D] fp32, positions offset..offset+S-1."""
    D = x.shape[-1]
    S = x.shape[-2]
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float32, device=x.device) / D))
    pos = torch.arange(offset, offset + S, dtype=torch.float32, device=x.device)
    fr = torch.outer(pos, inv)
    emb = torch.cat([fr, fr], dim=-1)
    cos, sin = emb.cos(), emb.sin()
    x1, x2 = x[..., : D // 2], x[..., D // 2:]
    rot = torch.cat([-x2, x1], dim=-1)
    return x * cos + rot * sin


def make_qkv(B=1, H=2, S_q=256, S_k=None, D=96, dtype=torch.bfloat16, seed=0,
             use_rope=True, sink_scale=None):
    """Q, K, V ~ N(0, 1) from a CPU generator (order q, k, v), RoPE on Q/K in
    fp32, optional K rows 0-3 scaled by ``sink_scale``, cast to ``dtype``.
    Returns CPU tensors."""
    S_k = S_q if S_k is None else S_k
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, H, S_q, D, generator=g)
    k = torch.randn(B, H, S_k, D, generator=g)
    v = torch.randn(B, H, S_k, D, generator=g)
    if use_rope:
        q = rope(q, offset=S_k - S_q)
        k = rope(k)
    if sink_scale is not None:
        k[:, :, :4] *= sink_scale
    return q.to(dtype), k.to(dtype), v.to(dtype)


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float32).numpy()


def dtype_tag(dtype: torch.dtype) -> str:
    return {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[dtype]
