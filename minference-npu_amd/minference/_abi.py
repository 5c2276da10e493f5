"""ctypes binding of libmsa.so (C ABI declared in include/msa.h).

The library is loaded from ``minference/_lib/libmsa.so`` (built in-tree by
``minference._build``).  There is no fallback: if the library or a GPU is
missing, every op raises.  Torch is used only to own device memory and to
name the current HIP stream.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional, Sequence

import torch

from ._build import LIB_PATH

# status codes (include/msa.h)
MSA_OK = 0
MSA_E_NULL = -1
MSA_E_RANK = -2
MSA_E_DTYPE = -3
MSA_E_HEAD_DIM = -4
MSA_E_ALIGN = -5
MSA_E_BLOCK = -6
MSA_E_TOPK = -7
MSA_E_HEADS = -8
MSA_E_WORKSPACE = -9
MSA_E_SEQ = -10
MSA_E_SLOTS = -11
MSA_E_SCRATCH = -12
MSA_E_FLAGS = -13
MSA_DECODE_SCRATCH_BYTES = 4 << 20

MSA_DTYPE_BF16 = 1
MSA_DTYPE_FP16 = 2
MSA_DTYPE_FP32 = 3

MSA_KIND_DENSE = 0
MSA_KIND_STREAM = 1
MSA_KIND_BLOCK = 2
MSA_KIND_VS = 3
MSA_KIND_FULL = 4
MSA_KIND_SKIP = 5
MSA_VS_MAX_SEQ = 131072

MSA_SELECT_FORCE_FIRST = 1
MSA_SELECT_FORCE_DIAG = 2
MSA_ESTIMATE_POOL_ONLY = 4
MSA_ESTIMATE_SELECT_ONLY = 8

MSA_MAX_HEADS = 128
MSA_BLOCK = 64
ABI_VERSION = 12

_DTYPE_CODE = {
    torch.bfloat16: MSA_DTYPE_BF16,
    torch.float16: MSA_DTYPE_FP16,
    torch.float32: MSA_DTYPE_FP32,
}

# every symbol include/msa.h declares
EXPORTED_SYMBOLS = (
    "msa_abi_version",
    "msa_status_str",
    "msa_estimate_workspace_bytes",
    "msa_block_estimate",
    "msa_block_estimate_ex",
    "msa_attention_workspace_bytes",
    "msa_layer_attention",
    "msa_stage_kv",
    "msa_layer_attention_staged",
    "msa_stage_kv_pool",
    "msa_decode_workspace_bytes",
    "msa_decode_attention",
    "msa_decode_attention_noalloc",
    "msa_vs_workspace_bytes",
    "msa_layer_attention_ex",
    "msa_vs_estimate_workspace_bytes",
    "msa_vs_estimate",
    "msa_rope_qk",
)


class MsaTensor4(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("size", ctypes.c_int64 * 4),
        ("stride", ctypes.c_int64 * 4),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class MsaHeadDesc(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("p1", ctypes.c_int32),
        ("p2", ctypes.c_int32),
        ("slot", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


class MsaVsLists(ctypes.Structure):
    _fields_ = [
        ("v_idx", ctypes.c_void_p),
        ("v_cnt", ctypes.c_void_p),
        ("s_idx", ctypes.c_void_p),
        ("s_cnt", ctypes.c_void_p),
        ("n_slots", ctypes.c_int32),
        ("v_stride", ctypes.c_int32),
        ("s_stride", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class MsaError(RuntimeError):
    """Raised for a non-zero status from libmsa."""

    def __init__(self, status: int, message: str):
        super().__init__(f"libmsa status {status}: {message}")
        self.status = status


_LIB = None
_LIB_LOCK = threading.Lock()


def library_path() -> str:
    """libmsa.so next to the package, or the build named by MINFERENCE_MSA_LIB."""
    return os.environ.get("MINFERENCE_MSA_LIB") or LIB_PATH


def load_library() -> ctypes.CDLL:
    """Load libmsa.so once; raises ImportError with the build command if absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LIB_LOCK:
        if _LIB is not None:
            return _LIB
        path = library_path()
        if not os.path.exists(path):
            raise ImportError(
                f"libmsa.so not found at {path}; build it with "
                "`python -m minference._build` (run from minference-npu_amd/)"
            )
        lib = ctypes.CDLL(path)
        lib.msa_abi_version.restype = ctypes.c_int
        lib.msa_abi_version.argtypes = []
        lib.msa_status_str.restype = ctypes.c_char_p
        lib.msa_status_str.argtypes = [ctypes.c_int]
        lib.msa_estimate_workspace_bytes.restype = ctypes.c_size_t
        lib.msa_estimate_workspace_bytes.argtypes = [
            ctypes.c_int64, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
        ]
        lib.msa_block_estimate.restype = ctypes.c_int
        lib.msa_block_estimate.argtypes = [
            ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
            ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.msa_block_estimate_ex.restype = ctypes.c_int
        lib.msa_block_estimate_ex.argtypes = [
            ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
            ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32),
            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_float, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.msa_attention_workspace_bytes.restype = ctypes.c_size_t
        lib.msa_attention_workspace_bytes.argtypes = [
            ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
        ]
        for name in ("msa_layer_attention", "msa_layer_attention_staged"):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [
                ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
                ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
                ctypes.POINTER(MsaHeadDesc), ctypes.c_int32,
                ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
            ]
        lib.msa_stage_kv.restype = ctypes.c_int
        lib.msa_stage_kv.argtypes = [
            ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.msa_stage_kv_pool.restype = ctypes.c_int
        lib.msa_stage_kv_pool.argtypes = [
            ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
            ctypes.POINTER(ctypes.c_int32), ctypes.c_int32,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.msa_decode_workspace_bytes.restype = ctypes.c_size_t
        lib.msa_decode_workspace_bytes.argtypes = [
            ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32,
        ]
        lib.msa_decode_attention.restype = ctypes.c_int
        lib.msa_decode_attention.argtypes = [
            ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
            ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
            ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.msa_decode_attention_noalloc.restype = ctypes.c_int
        lib.msa_decode_attention_noalloc.argtypes = [
            ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
            ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
            ctypes.c_float, ctypes.c_void_p,
        ]
        lib.msa_vs_estimate_workspace_bytes.restype = ctypes.c_size_t
        lib.msa_vs_estimate_workspace_bytes.argtypes = [
            ctypes.c_int64, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
        ]
        lib.msa_vs_estimate.restype = ctypes.c_int
        lib.msa_vs_estimate.argtypes = [
            ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
        ]
        lib.msa_vs_workspace_bytes.restype = ctypes.c_size_t
        lib.msa_vs_workspace_bytes.argtypes = [
            ctypes.c_int64, ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
        ]
        lib.msa_layer_attention_ex.restype = ctypes.c_int
        lib.msa_layer_attention_ex.argtypes = [
            ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
            ctypes.POINTER(MsaTensor4), ctypes.POINTER(MsaTensor4),
            ctypes.POINTER(MsaHeadDesc), ctypes.c_int32,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
            ctypes.POINTER(MsaVsLists), ctypes.c_void_p, ctypes.c_size_t,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_void_p,
        ]
        lib.msa_rope_qk.restype = ctypes.c_int
        lib.msa_rope_qk.argtypes = [ctypes.POINTER(MsaTensor4)] * 6 + [ctypes.c_void_p]
        ver = lib.msa_abi_version()
        if ver != ABI_VERSION:
            raise ImportError(f"libmsa ABI version {ver} != expected {ABI_VERSION}")
        _LIB = lib
        return lib


def status_str(status: int) -> str:
    return load_library().msa_status_str(int(status)).decode()


def check(status: int) -> None:
    if status == MSA_OK:
        return
    msg = status_str(status)
    if status < 0:
        raise ValueError(f"libmsa rejected the call (status {status}): {msg}")
    raise MsaError(status, msg)


def tensor4(t: torch.Tensor) -> MsaTensor4:
    if t.dim() != 4:
        raise ValueError(f"expected a 4-D [B,H,S,D] tensor, got {t.dim()}-D")
    code = _DTYPE_CODE.get(t.dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {t.dtype}")
    d = MsaTensor4()
    d.data = t.data_ptr()
    for i in range(4):
        d.size[i] = int(t.shape[i])
        d.stride[i] = int(t.stride(i))
    d.dtype = code
    return d


def require_device(*tensors: torch.Tensor) -> None:
    """The MI355X path has no CPU fallback: inputs must live on the GPU."""
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                "minference (MI355X build) runs on the GPU only; got a tensor on "
                f"{t.device}.  Move q/k/v to the HIP device."
            )
    dev = tensors[0].device
    for t in tensors[1:]:
        if t.device != dev:
            raise RuntimeError("q, k and v must be on the same device")


def current_stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def estimate_workspace_bytes(batch: int, n_slots: int, s_q: int, s_k: int, head_dim: int) -> int:
    return int(load_library().msa_estimate_workspace_bytes(batch, n_slots, s_q, s_k, head_dim))


def attention_workspace_bytes(batch: int, kv_heads: int, s_k: int, head_dim: int) -> int:
    return int(load_library().msa_attention_workspace_bytes(batch, kv_heads, s_k, head_dim))


def decode_workspace_bytes(batch: int, heads: int, s_k: int, head_dim: int) -> int:
    return int(load_library().msa_decode_workspace_bytes(batch, heads, s_k, head_dim))


def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                     scale: float, ws: Optional[torch.Tensor] = None) -> None:
    """Launch msa_decode_attention (q [B,H,1,D] against the cache k/v) on the
    current stream."""
    need = decode_workspace_bytes(q.shape[0], q.shape[1], k.shape[2], q.shape[3])
    if ws is None or ws.numel() < need:
        ws = workspace(need, q.device)
    qd, kd, vd, od = tensor4(q), tensor4(k), tensor4(v), tensor4(out)
    check(load_library().msa_decode_attention(
        ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), ctypes.byref(od), float(scale),
        ws.data_ptr(), ws.numel(), current_stream_handle(q.device)))


def decode_attention_noalloc(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                             out: torch.Tensor, scale: float) -> None:
    """Launch msa_decode_attention_noalloc on the current stream: the same
    decode as decode_attention with the partials in the library's fixed
    per-GPU scratch (no workspace, nothing allocated)."""
    qd, kd, vd, od = tensor4(q), tensor4(k), tensor4(v), tensor4(out)
    check(load_library().msa_decode_attention_noalloc(
        ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), ctypes.byref(od), float(scale),
        current_stream_handle(q.device)))


def rope_qk(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
            q_out: torch.Tensor, k_out: torch.Tensor) -> None:
    """Launch msa_rope_qk on the current stream: q [B,H,S,D], k [B,H_kv,S,D],
    cos/sin [B or 1, 1, S, rot] views; q_out/k_out may be q/k (in place)."""
    require_device(q, k, cos, sin, q_out, k_out)
    ds = [tensor4(t) for t in (q, k, cos, sin, q_out, k_out)]
    check(load_library().msa_rope_qk(*[ctypes.byref(d) for d in ds],
                                     current_stream_handle(q.device)))


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Caller-owned workspace (256-byte aligned by the caching allocator)."""
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def block_estimate(
    q: torch.Tensor,
    k: torch.Tensor,
    slot_heads: Sequence[int],
    slot_topk: Sequence[int],
    topk_max: int,
    score_scale: float,
    idx: torch.Tensor,
    cnt: torch.Tensor,
    ws: Optional[torch.Tensor] = None,
    flags: int = 0,
    block: int = MSA_BLOCK,
) -> None:
    """Launch msa_block_estimate on the current stream (no sync); with
    ``flags`` (MSA_SELECT_* / MSA_ESTIMATE_*) msa_block_estimate_ex.  The
    one-pass flags need the caller's workspace (the select pass reads what
    the pooling pass left in it).  ``block``: tokens per block (64, 128, 256
    or 512); idx / cnt are in those blocks."""
    lib = load_library()
    n_slots = len(slot_heads)
    if len(slot_topk) != n_slots:
        raise ValueError("slot_topk must have one entry per slot")
    heads_arr = (ctypes.c_int32 * max(n_slots, 1))(*[int(h) for h in slot_heads])
    topk_arr = (ctypes.c_int32 * max(n_slots, 1))(*[int(t) for t in slot_topk])
    need = estimate_workspace_bytes(q.shape[0], n_slots, q.shape[2], k.shape[2], q.shape[3])
    if ws is None or ws.numel() < need:
        if flags & (MSA_ESTIMATE_POOL_ONLY | MSA_ESTIMATE_SELECT_ONLY):
            raise ValueError("a one-pass block estimate needs the caller's workspace "
                             f"of at least {need} bytes")
        ws = workspace(need, q.device)
    qd, kd = tensor4(q), tensor4(k)
    stream = current_stream_handle(q.device)
    if flags:
        st = lib.msa_block_estimate_ex(
            ctypes.byref(qd), ctypes.byref(kd), heads_arr, topk_arr, n_slots, int(block),
            int(topk_max), float(score_scale), int(flags), idx.data_ptr(), cnt.data_ptr(),
            ws.data_ptr(), ws.numel(), stream)
    else:
        st = lib.msa_block_estimate(
            ctypes.byref(qd), ctypes.byref(kd), heads_arr, topk_arr, n_slots, int(block),
            int(topk_max), float(score_scale), idx.data_ptr(), cnt.data_ptr(), ws.data_ptr(),
            ws.numel(), stream)
    check(st)


def head_descs(heads: Sequence[tuple]):
    """ctypes array of msa_head_desc from [(kind, p1, p2, slot, scale)]."""
    n = len(heads)
    arr = (MsaHeadDesc * max(n, 1))()
    for i, (kind, p1, p2, slot, scale) in enumerate(heads):
        arr[i].kind = int(kind)
        arr[i].p1 = int(p1)
        arr[i].p2 = int(p2)
        arr[i].slot = int(slot)
        arr[i].scale = float(scale)
    return arr


def stage_kv(k: torch.Tensor, v: torch.Tensor, ws: torch.Tensor) -> None:
    """Launch msa_stage_kv (K, V -> MFMA operand order in ``ws``) on the
    current stream."""
    kd, vd = tensor4(k), tensor4(v)
    check(load_library().msa_stage_kv(ctypes.byref(kd), ctypes.byref(vd), ws.data_ptr(),
                                      ws.numel(), current_stream_handle(v.device)))


def stage_kv_pool(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  slot_heads: Sequence[int], est_ws: Optional[torch.Tensor],
                  ws: torch.Tensor) -> None:
    """Launch msa_stage_kv_pool on the current stream: V (and K where the
    attention kernel cannot read it in place) staged into ``ws`` and, for the block slots ``slot_heads``, Q and K pooled into ``est_ws``
    (the workspace of the MSA_ESTIMATE_SELECT_ONLY block_estimate call that
    follows)."""
    n = len(slot_heads)
    heads_arr = (ctypes.c_int32 * max(n, 1))(*[int(h) for h in slot_heads])
    qd, kd, vd = tensor4(q), tensor4(k), tensor4(v)
    est_p = est_ws.data_ptr() if est_ws is not None else None
    est_n = est_ws.numel() if est_ws is not None else 0
    check(load_library().msa_stage_kv_pool(
        ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), heads_arr, n, est_p, est_n,
        ws.data_ptr(), ws.numel(), current_stream_handle(v.device)))


def vs_estimate_workspace_bytes(batch: int, n_slots: int, s: int, head_dim: int) -> int:
    return int(load_library().msa_vs_estimate_workspace_bytes(batch, n_slots, s, head_dim))


def vs_estimate(q: torch.Tensor, k: torch.Tensor, slot_heads: Sequence[int],
                slot_vsize: Sequence[int], slot_ssize: Sequence[int], v_idx: torch.Tensor,
                v_cnt: torch.Tensor, s_idx: torch.Tensor, s_cnt: torch.Tensor,
                ws: Optional[torch.Tensor] = None) -> None:
    """Launch msa_vs_estimate on the current stream: v_idx [B,slots,v_stride],
    s_idx [B,slots,s_stride], v_cnt / s_cnt [B,slots], int32 contiguous."""
    lib = load_library()
    n = len(slot_heads)
    for t in (v_idx, v_cnt, s_idx, s_cnt):
        if t.dtype != torch.int32 or not t.is_contiguous() or t.device != q.device:
            raise ValueError("vertical_and_slash lists must be contiguous int32 on q's device")
    heads_arr = (ctypes.c_int32 * max(n, 1))(*[int(h) for h in slot_heads])
    v_arr = (ctypes.c_int32 * max(n, 1))(*[int(x) for x in slot_vsize])
    s_arr = (ctypes.c_int32 * max(n, 1))(*[int(x) for x in slot_ssize])
    need = vs_estimate_workspace_bytes(q.shape[0], n, q.shape[2], q.shape[3])
    if ws is None or ws.numel() < need:
        ws = workspace(need, q.device)
    qd, kd = tensor4(q), tensor4(k)
    check(lib.msa_vs_estimate(
        ctypes.byref(qd), ctypes.byref(kd), heads_arr, v_arr, s_arr, n,
        v_idx.data_ptr(), v_cnt.data_ptr(), int(v_idx.shape[-1]),
        s_idx.data_ptr(), s_cnt.data_ptr(), int(s_idx.shape[-1]),
        ws.data_ptr(), ws.numel(), current_stream_handle(q.device)))


def vs_workspace_bytes(batch: int, n_slots: int, s_k: int, v_stride: int, head_dim: int) -> int:
    return int(load_library().msa_vs_workspace_bytes(batch, n_slots, s_k, v_stride, head_dim))


def layer_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    heads: Sequence[tuple],
    idx: Optional[torch.Tensor] = None,
    cnt: Optional[torch.Tensor] = None,
    idx_slots: int = 0,
    topk_max: int = 0,
    ws: Optional[torch.Tensor] = None,
    staged: bool = False,
    vs: Optional[tuple] = None,
    vs_ws: Optional[torch.Tensor] = None,
) -> None:
    """Launch msa_layer_attention (or, with ``staged=True``,
    msa_layer_attention_staged reading what msa_stage_kv staged in ``ws``
    for the same k and v).
    ``heads`` = [(kind, p1, p2, slot, scale)] * H.  With vertical_and_slash
    heads, ``vs`` = (v_idx [B,slots,nv], v_cnt [B,slots], s_idx [B,slots,ns],
    s_cnt [B,slots]) int32 contiguous device tensors and the call goes to
    msa_layer_attention_ex."""
    lib = load_library()
    n = len(heads)
    arr = head_descs(heads)
    need = attention_workspace_bytes(k.shape[0], k.shape[1], k.shape[2], k.shape[3])
    if staged and (ws is None or ws.numel() < need):
        raise ValueError("staged attention needs the workspace filled by stage_kv")
    if ws is None or ws.numel() < need:
        ws = workspace(need, q.device)
    for t in (idx, cnt):
        if t is not None and (t.dtype != torch.int32 or not t.is_contiguous()
                              or t.device != q.device):
            raise ValueError("block ids / counts must be contiguous int32 on q's device")
    qd, kd, vd, od = tensor4(q), tensor4(k), tensor4(v), tensor4(out)
    idx_p = idx.data_ptr() if idx is not None else None
    cnt_p = cnt.data_ptr() if cnt is not None else None
    stream = current_stream_handle(q.device)
    if vs is not None:
        v_idx, v_cnt, s_idx, s_cnt = vs
        for t in vs:
            if t.dtype != torch.int32 or not t.is_contiguous() or t.device != q.device:
                raise ValueError("vertical_and_slash lists must be contiguous int32 on q's device")
        lists = MsaVsLists(v_idx.data_ptr(), v_cnt.data_ptr(), s_idx.data_ptr(), s_cnt.data_ptr(),
                           int(v_idx.shape[1]), int(v_idx.shape[2]), int(s_idx.shape[2]), 0)
        vneed = vs_workspace_bytes(q.shape[0], v_idx.shape[1], k.shape[2], v_idx.shape[2],
                                   q.shape[3])
        if vs_ws is None or vs_ws.numel() < vneed:
            vs_ws = workspace(vneed, q.device)
        st = lib.msa_layer_attention_ex(
            ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), ctypes.byref(od), arr, n,
            idx_p, cnt_p, int(idx_slots), int(topk_max), ctypes.byref(lists),
            vs_ws.data_ptr(), vs_ws.numel(), ws.data_ptr(), ws.numel(), 0 if staged else 1,
            stream)
        check(st)
        return
    fn = lib.msa_layer_attention_staged if staged else lib.msa_layer_attention
    st = fn(
        ctypes.byref(qd), ctypes.byref(kd), ctypes.byref(vd), ctypes.byref(od),
        arr, n, idx_p, cnt_p,
        int(idx_slots), int(topk_max), ws.data_ptr(), ws.numel(),
        stream,
    )
    check(st)
