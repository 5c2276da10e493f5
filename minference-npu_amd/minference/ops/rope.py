"""Rotary position embedding of a layer's q and k heads in one HIP launch.

Replaces the apply_rotary_pos_emb call of the patched forward (reference
minference/modules/minference_forward.py:205-212 looks up the model
module's function, :336-341 calls it): HF's rotate-half form
``q * cos + rotate_half(q) * sin`` on the first ``rot = cos.shape[-1]`` dims,
the rest passed through.  Every product and sum is rounded to the input
dtype as the eager elementwise ops round them, so the result is bit-identical
to the HF function, in one pass over q and k instead of about ten.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _abi

__all__ = ["apply_rotary_pos_emb", "rope_supported"]

_DTYPES = (torch.bfloat16, torch.float16)


def rope_supported(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> bool:
    """True when msa_rope_qk takes these tensors: GPU, bf16/fp16 throughout,
    q/k [B, H, S, D] views with D contiguous, cos/sin [B or 1, S, rot] with
    rot % 16 == 0, rot <= D, D % 8 == 0, 16-byte aligned rows."""
    ts = (q, k, cos, sin)
    if not all(t.is_cuda for t in ts) or q.dtype not in _DTYPES:
        return False
    if any(t.dtype != q.dtype for t in ts) or q.dim() != 4 or k.dim() != 4 or cos.dim() != 3:
        return False
    B, _, S, D = q.shape
    rot = cos.shape[-1]
    if sin.shape != cos.shape or cos.shape[0] not in (1, B) or cos.shape[1] != S:
        return False
    if k.shape[0] != B or k.shape[2] != S or k.shape[3] != D:
        return False
    if D % 8 or rot % 16 or rot > D:
        return False
    for t in ts:
        if t.stride(-1) != 1 or t.data_ptr() % 16:
            return False
        if any(t.stride(i) * t.element_size() % 16 for i in range(t.dim() - 1) if t.shape[i] > 1):
            return False
    return True


def apply_rotary_pos_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
                         sin: torch.Tensor, unsqueeze_dim: int = 1, *,
                         inplace: bool = False,
                         out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None):
    """HF's ``apply_rotary_pos_emb(q, k, cos, sin)`` on the GPU.

    Args:
        q, k:      ``[B, H, S, D]`` / ``[B, H_kv, S, D]`` (views of a fused qkv
                   projection are read in place).
        cos, sin:  ``[B or 1, S, rot]`` position tables in q's dtype.
        unsqueeze_dim: must be 1 (the head axis), as in the BNSD forward.
        inplace:   write the result into q and k and return them.
        out:       optional (q_out, k_out) to write into.

    Returns (q_embed, k_embed).  Without ``inplace`` / ``out`` the outputs are
    new ``[B, H, S, D]`` views over ``[B, S, H, D]`` memory (one token's heads
    adjacent, the order the kernel writes in).
    """
    if unsqueeze_dim != 1:
        raise NotImplementedError("only unsqueeze_dim=1 ([B, H, S, D] q/k) is supported")
    if not rope_supported(q, k, cos, sin):
        raise NotImplementedError(
            "msa_rope_qk needs GPU bf16/fp16 tensors, q/k [B,H,S,D] and cos/sin "
            f"[B|1,S,rot] with rot % 16 == 0 and rot <= D % 8 == 0; got q={tuple(q.shape)} "
            f"{q.dtype} {q.device}, cos={tuple(cos.shape)} {cos.dtype}")
    if inplace:
        qo, ko = q, k
    elif out is not None:
        qo, ko = out
    else:
        B, H, S, D = q.shape
        qo = torch.empty((B, S, H, D), dtype=q.dtype, device=q.device).transpose(1, 2)
        ko = torch.empty((B, S, k.shape[1], D), dtype=k.dtype, device=k.device).transpose(1, 2)
    _abi.rope_qk(q, k, cos[:, None], sin[:, None], qo, ko)
    return qo, ko
