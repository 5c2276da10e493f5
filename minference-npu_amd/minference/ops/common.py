"""Shared host helpers for the MI355X ops (argument checks, scale rule, output)."""

from __future__ import annotations

import functools
import inspect
import math
from typing import Optional, Sequence

import torch

from .. import _abi

# Head dims the reference pads to before computing the sparse-op scale
# (minference/ops/streaming_kernel_npu.py:70-86; block_sparse_kernel_npu.py:56, 95-101).
ALLOWED_HEAD_DIMS = (16, 32, 64, 128, 256, 512)

# Head dims the HIP kernels are built for; the ops take any head_dim up to the
# largest of them by zero-padding q, k and v to the next one.
SUPPORTED_HEAD_DIMS = (64, 96, 128, 256, 512)
# vertical_and_slash (estimator and attention) is built up to 128
VS_HEAD_DIMS = (64, 96, 128)
SUPPORTED_DTYPES = (torch.bfloat16, torch.float16)


def sixteen_bit_dtype(tensors: Sequence[torch.Tensor]) -> torch.dtype:
    """The 16-bit type float32 op inputs are rounded to on the device: fp16
    (11 significant bits) when every finite value lies within its range,
    else bf16; non-finite values stay non-finite in either."""
    lim = torch.finfo(torch.float16).max
    for t in tensors:
        if t.numel() and float(torch.where(torch.isfinite(t), t.abs(), 0.0).amax()) > lim:
            return torch.bfloat16
    return torch.float16


def accepts_float32(names: Sequence[str], has_out: bool = True):
    """Decorator for the public ops: called with float32 tensors ``names``,
    the op runs on their on-device roundings to sixteen_bit_dtype and, when
    it has an output, writes it in float32 (``out`` must then be float32 or
    None).  The reference's CPU paths take any float dtype and compute in
    fp32 (minference/ops/streaming_kernel_npu.py:138-144,
    minference/ops/block_sparse_kernel_npu.py:340-348); here float32 inputs
    get the 16-bit kernels' arithmetic on their roundings.  Inputs of other
    dtypes go to the op unchanged (bf16 / fp16, or its dtype error)."""

    def wrap(fn):
        sig = inspect.signature(fn)

        @functools.wraps(fn)
        def inner(*args, **kwargs):
            ba = sig.bind(*args, **kwargs)
            ts = [ba.arguments.get(n) for n in names]
            if not all(isinstance(t, torch.Tensor) and t.dtype == torch.float32 for t in ts):
                return fn(*args, **kwargs)
            dt = sixteen_bit_dtype(ts)
            for n, t in zip(names, ts):
                ba.arguments[n] = t.to(dt)
            if has_out:
                out = ba.arguments.get("out")
                if out is None:
                    ba.arguments["out"] = torch.empty(ts[0].shape, dtype=torch.float32,
                                                      device=ts[0].device)
                elif out.dtype != torch.float32:
                    raise ValueError(f"out must be float32 for float32 inputs, got {out.dtype}")
            return fn(*ba.args, **ba.kwargs)

        return inner

    return wrap


def next_allowed_head_dim(d: int) -> int:
    for cand in ALLOWED_HEAD_DIMS:
        if cand >= d:
            return cand
    raise ValueError(
        f"head_dim={d} exceeds the largest supported value {ALLOWED_HEAD_DIMS[-1]}"
    )


def sparse_scale(head_dim: int) -> float:
    """Scale of stream_llm / block_sparse heads.  The reference zero-pads
    head_dim to the next allowed size *before* computing 1/sqrt(D)
    (streaming_kernel_npu.py:114 after :377-381; block_sparse_kernel_npu.py:254,
    340 after :651-656), so Phi-3 (D=96) uses 128**-0.5.  Padding with zeros
    does not change q.k, so the kernels run on the unpadded D with this scale."""
    return next_allowed_head_dim(head_dim) ** -0.5


def dense_scale(head_dim: int) -> float:
    """dense_attention's default 1/sqrt(D), unpadded (backend_npu/attention.py:210-211)."""
    return 1.0 / math.sqrt(head_dim)


def check_bnsd(q: torch.Tensor, k: torch.Tensor, v: Optional[torch.Tensor] = None) -> None:
    """Rank / shape checks with the reference's AssertionError contract
    (streaming_kernel_npu.py:369-372, block_sparse_kernel_npu.py:640-643)."""
    assert q.dim() == 4, f"q must be 4-D [B,H,S,D], got {q.dim()}-D"
    assert (
        q.shape[0] == k.shape[0] and q.shape[1] == k.shape[1] and q.shape[-1] == k.shape[-1]
    ), f"q/k B/H/D mismatch; q={tuple(q.shape)} k={tuple(k.shape)}"
    if v is not None:
        assert v.shape == k.shape, f"v shape {tuple(v.shape)} != k shape {tuple(k.shape)}"


def kernel_head_dim(d: int) -> int:
    """The head dim the kernels run at for head_dim ``d``: d itself when the
    kernels are built for it, else the next built size.  The ops pad q, k and
    v with zeros to it (no dot product changes; the extra output columns are
    dropped), as the reference pads to its allowed sizes before its kernels
    (streaming_kernel_npu.py:377-381, block_sparse_kernel_npu.py:651-656).
    The scale still follows the reference's rule for the original d."""
    for cand in SUPPORTED_HEAD_DIMS:
        if cand >= d:
            return cand
    raise NotImplementedError(
        f"head_dim={d} is not supported by the MI355X kernels (at most "
        f"{SUPPORTED_HEAD_DIMS[-1]}; the reference pads up to {ALLOWED_HEAD_DIMS[-1]})"
    )


def require_kernel_head_dim(d: int, what: str, dims: Sequence[int] = SUPPORTED_HEAD_DIMS) -> None:
    """Paths that do not pad (vertical_and_slash, whose estimator divides by
    the kernel's sqrt(D) and is built up to 128; the patched model forward)
    take the built head dims only."""
    if d not in dims:
        raise NotImplementedError(f"{what} runs at head_dim {tuple(dims)} only, got {d}")


def pad_head_dim(t: torch.Tensor, dk: int) -> torch.Tensor:
    """t with its last dimension zero-padded to dk (t itself when it is dk)."""
    if t.shape[-1] == dk:
        return t
    return torch.nn.functional.pad(t, (0, dk - t.shape[-1]))


def padded_call(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: Optional[torch.Tensor],
                fn) -> torch.Tensor:
    """Run ``fn(q, k, v, result)`` on views the kernels read in place, at the
    kernel head dim; returns the op's output (``out`` when given) with the
    original head_dim."""
    d = q.shape[-1]
    dk = kernel_head_dim(d)
    result = make_out(q, out)
    if dk == d:
        fn(kernel_view(q), kernel_view(k), kernel_view(v), result)
        return result
    qp, kp, vp = pad_head_dim(q, dk), pad_head_dim(k, dk), pad_head_dim(v, dk)
    tmp = torch.empty(qp.shape, dtype=result.dtype, device=q.device)
    fn(qp, kp, vp, tmp)
    result.copy_(tmp[..., :d])
    return result


def check_supported(q: torch.Tensor, k: torch.Tensor, v: Optional[torch.Tensor] = None,
                    allow_longer_q: bool = False) -> None:
    tensors = (q, k) if v is None else (q, k, v)
    _abi.require_device(*tensors)
    for t in tensors:
        if t.dtype not in SUPPORTED_DTYPES:
            raise NotImplementedError(
                f"the MI355X kernels take bf16 or fp16 inputs, got {t.dtype}"
            )
    if len({t.dtype for t in tensors}) != 1:
        raise ValueError("q, k and v must share one dtype")
    if q.shape[-1] < 1:
        raise ValueError("head_dim must be positive")
    kernel_head_dim(q.shape[-1])  # NotImplementedError beyond the largest built size
    if q.shape[2] > k.shape[2] and not allow_longer_q:
        raise ValueError(
            f"prefill attention requires S_q <= S_k, got S_q={q.shape[2]}, S_k={k.shape[2]}"
        )


def kernel_view(t: torch.Tensor) -> torch.Tensor:
    """A view the kernels can read in place (D contiguous, 16-byte rows)."""
    if t.stride(-1) != 1 or (t.data_ptr() % 16) != 0 or any(
        (t.stride(i) * t.element_size()) % 16 for i in range(3) if t.shape[i] > 1
    ):
        return t.contiguous()
    return t


def make_out(q: torch.Tensor, out: Optional[torch.Tensor]) -> torch.Tensor:
    if out is None:
        return torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if out.shape != q.shape:
        raise ValueError(f"out shape {tuple(out.shape)} != q shape {tuple(q.shape)}")
    if out.dtype not in (q.dtype, torch.float32):
        raise ValueError(f"out dtype must be {q.dtype} or float32, got {out.dtype}")
    if out.device != q.device:
        raise ValueError("out must be on q's device")
    return out


def head_chunks(n_heads: int):
    """Head ranges of at most MSA_MAX_HEADS per library call."""
    step = _abi.MSA_MAX_HEADS
    for h0 in range(0, n_heads, step):
        yield h0, min(n_heads, h0 + step)
