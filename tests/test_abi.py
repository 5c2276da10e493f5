"""C ABI checks that need no GPU: the library loads, exports every function
include/msa.h declares, and rejects bad arguments before any launch."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from minference import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "msa.h")

FAKE = 0x10000  # never dereferenced: validation fails first


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(msa_\w+)\s*\(", text, flags=re.M)))


def test_header_lists_expected_functions():
    assert header_functions() == sorted(_abi.EXPORTED_SYMBOLS)


def test_library_exports_every_header_symbol():
    lib = _abi.load_library()
    for name in header_functions():
        assert hasattr(lib, name), name


def test_abi_version_and_status_strings():
    lib = _abi.load_library()
    assert lib.msa_abi_version() == _abi.ABI_VERSION
    for code in range(-13, 1):
        s = _abi.status_str(code)
        assert s and s != "unknown status"
    assert _abi.status_str(-99) == "unknown status"


def test_decode_noalloc_refuses_oversize_before_any_device_call():
    """The no-allocation decode rejects partials larger than its fixed
    scratch (fake pointers: nothing is dereferenced or launched)."""
    lib = _abi.load_library()
    bh = 20000  # one split per head: 20000 * 130 * 4 bytes > 4 MiB at D = 128
    assert _abi.decode_workspace_bytes(1, bh, 4096, 128) > _abi.MSA_DECODE_SCRATCH_BYTES
    q, kv = t4([1, bh, 1, 128]), t4([1, bh, 4096, 128])
    st = lib.msa_decode_attention_noalloc(ctypes.byref(q), ctypes.byref(kv), ctypes.byref(kv),
                                          ctypes.byref(q), 0.088, None)
    assert st == _abi.MSA_E_SCRATCH
    assert "scratch" in _abi.status_str(st)


def test_workspace_sizes():
    # estimator: pooled Q (rows padded to 16) and pooled K in the input dtype,
    # then the fp32 pooled scores of every (padded) row, rows padded to 16
    # candidates; each part rounded up to 256 bytes
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    assert _abi.estimate_workspace_bytes(1, 32, 16384, 16384, 96) == \
        up(32 * 256 * 96 * 2) + up(32 * 256 * 96 * 2) + up(32 * 256 * 256 * 4)
    assert _abi.estimate_workspace_bytes(1, 1, 100, 100, 64) == \
        up(16 * 64 * 2) + up(2 * 64 * 2) + up(16 * 16 * 4)
    # attention: staged K and V operands (16-bit) padded to 64 keys, the V
    # maxima per 64-key tile (fp32) and the V exponent per kv head (int32),
    # each rounded up to 256 bytes, then 256 bytes of work-queue counters
    staged = 2 * 32 * 96 * 65536 * 2
    assert _abi.attention_workspace_bytes(1, 32, 65536, 96) == \
        up(up(staged + 32 * 1024 * 4) + 32 * 4) + 256
    assert _abi.attention_workspace_bytes(1, 1, 65, 64) == up(up(2 * 64 * 128 * 2 + 2 * 4) + 4) + 256
    assert _abi.attention_workspace_bytes(0, 1, 65, 64) == 0


def t4(shape, dtype=_abi.MSA_DTYPE_BF16, strides=None, data=FAKE):
    d = _abi.MsaTensor4()
    d.data = data
    if strides is None:
        strides = [shape[1] * shape[2] * shape[3], shape[2] * shape[3], shape[3], 1]
    for i in range(4):
        d.size[i] = shape[i]
        d.stride[i] = strides[i]
    d.dtype = dtype
    return d


def heads(n, kind=_abi.MSA_KIND_STREAM, slot=-1, scale=0.088):
    arr = (_abi.MsaHeadDesc * n)()
    for i in range(n):
        arr[i].kind = kind
        arr[i].p1 = 64
        arr[i].p2 = 256
        arr[i].slot = slot if slot >= 0 else -1
        arr[i].scale = scale
    return arr


def attn(q, k, v, o, hd, n, idx=None, cnt=None, slots=0, topk=0, ws=FAKE, wsb=1 << 40):
    lib = _abi.load_library()
    return lib.msa_layer_attention(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v),
                                   ctypes.byref(o), hd, n, idx, cnt, slots, topk, ws, wsb, None)


def est(q, k, heads_list, topk_list, topk_max, scale=0.088, block=64, ws=FAKE, wsb=1 << 40,
        idx=FAKE, cnt=FAKE):
    lib = _abi.load_library()
    n = len(heads_list)
    ha = (ctypes.c_int32 * max(n, 1))(*heads_list)
    ta = (ctypes.c_int32 * max(n, 1))(*topk_list) if topk_list is not None else None
    return lib.msa_block_estimate(ctypes.byref(q), ctypes.byref(k), ha, ta, n, block, topk_max,
                                  scale, idx, cnt, ws, wsb, None)


SHAPE = [1, 4, 256, 96]


@pytest.mark.parametrize(
    "mutate,expected",
    [
        (lambda a: a.__setitem__("q", t4([1, 4, 256, 80])), _abi.MSA_E_RANK),
        (lambda a: a.__setitem__("q", t4([1, 4, 256, 48]))
         or a.__setitem__("k", t4([1, 4, 256, 48])) or a.__setitem__("v", t4([1, 4, 256, 48]))
         or a.__setitem__("o", t4([1, 4, 256, 48])), _abi.MSA_E_HEAD_DIM),
        (lambda a: a.__setitem__("q", t4(SHAPE, _abi.MSA_DTYPE_FP32)), _abi.MSA_E_DTYPE),
        (lambda a: a.__setitem__("o", t4(SHAPE, _abi.MSA_DTYPE_FP16)), _abi.MSA_E_DTYPE),
        (lambda a: a.__setitem__("k", t4(SHAPE, strides=[4 * 256 * 96, 256 * 96, 96, 2])), _abi.MSA_E_ALIGN),
        (lambda a: a.__setitem__("q", t4(SHAPE, strides=[4 * 256 * 100, 256 * 100, 100, 1])), _abi.MSA_E_ALIGN),
        (lambda a: a.__setitem__("q", t4(SHAPE, data=FAKE + 2)), _abi.MSA_E_ALIGN),
        (lambda a: a.__setitem__("q", t4(SHAPE, strides=[4 * 256 << 24, 256 << 24, 1 << 24, 1])),
         _abi.MSA_E_ALIGN),
        (lambda a: a.__setitem__("q", t4([1, 4, 512, 96])) or a.__setitem__("o", t4([1, 4, 512, 96])), _abi.MSA_E_SEQ),
        (lambda a: a.__setitem__("n", 3), _abi.MSA_E_HEADS),
        (lambda a: a.__setitem__("hd", heads(4, kind=7)), _abi.MSA_E_HEADS),
        (lambda a: a.__setitem__("hd", heads(4, scale=0.0)), _abi.MSA_E_HEADS),
        (lambda a: a.__setitem__("hd", heads(4, kind=_abi.MSA_KIND_BLOCK, slot=0)), _abi.MSA_E_SLOTS),
        (lambda a: a.__setitem__("wsb", 100), _abi.MSA_E_WORKSPACE),
        (lambda a: a.__setitem__("ws", None), _abi.MSA_E_WORKSPACE),
        (lambda a: a.__setitem__("q", t4(SHAPE, data=0)), _abi.MSA_E_NULL),
        (lambda a: a.__setitem__("k", t4([1, 3, 256, 96])) or a.__setitem__("v", t4([1, 3, 256, 96])), _abi.MSA_E_RANK),
    ],
)
def test_attention_validation(mutate, expected):
    a = {"q": t4(SHAPE), "k": t4(SHAPE), "v": t4(SHAPE), "o": t4(SHAPE), "hd": heads(4), "n": 4,
         "ws": FAKE, "wsb": 1 << 40}
    mutate(a)
    assert attn(a["q"], a["k"], a["v"], a["o"], a["hd"], a["n"], ws=a["ws"], wsb=a["wsb"]) == expected


def test_head_dim_256_accepted_and_vs_refused():
    """D = 256 and 512 pass the attention and estimator checks (failing later, on
    the deliberately small workspace); 160 is refused; vertical_and_slash
    (estimator and attention) stays at D <= 128."""
    lib = _abi.load_library()
    d256 = [1, 4, 256, 256]
    assert attn(t4(d256), t4(d256), t4(d256), t4(d256), heads(4), 4, wsb=100) == _abi.MSA_E_WORKSPACE
    d512 = [1, 4, 256, 512]
    assert attn(t4(d512), t4(d512), t4(d512), t4(d512), heads(4), 4, wsb=100) == _abi.MSA_E_WORKSPACE
    d160 = [1, 4, 256, 160]
    assert attn(t4(d160), t4(d160), t4(d160), t4(d160), heads(4), 4) == _abi.MSA_E_HEAD_DIM
    assert est(t4(d256), t4(d256), [0], [2], 2, wsb=100) == _abi.MSA_E_WORKSPACE
    one = (ctypes.c_int32 * 1)(0)
    sz = (ctypes.c_int32 * 1)(30)
    st = lib.msa_vs_estimate(ctypes.byref(t4(d256)), ctypes.byref(t4(d256)), one, sz, sz, 1,
                             FAKE, FAKE, 64, FAKE, FAKE, 64, FAKE, 1 << 40, None)
    assert st == _abi.MSA_E_HEAD_DIM
    vs_heads = heads(4, kind=_abi.MSA_KIND_VS, slot=0)
    assert attn(t4(d256), t4(d256), t4(d256), t4(d256), vs_heads, 4) == _abi.MSA_E_HEAD_DIM


def test_attention_full_kind_allows_longer_queries():
    """S_q > S_k is refused for causal kinds and accepted for MSA_KIND_FULL
    heads (the call then fails later, on the deliberately small workspace)."""
    q, kv = t4([1, 4, 512, 96]), t4([1, 4, 256, 96])
    assert attn(q, kv, kv, q, heads(4), 4, wsb=100) == _abi.MSA_E_SEQ
    assert attn(q, kv, kv, q, heads(4, kind=_abi.MSA_KIND_DENSE), 4, wsb=100) == _abi.MSA_E_SEQ
    assert attn(q, kv, kv, q, heads(4, kind=_abi.MSA_KIND_FULL), 4, wsb=100) == _abi.MSA_E_WORKSPACE
    mixed = heads(4, kind=_abi.MSA_KIND_FULL)
    mixed[2].kind = _abi.MSA_KIND_STREAM
    assert attn(q, kv, kv, q, mixed, 4, wsb=100) == _abi.MSA_E_SEQ


def test_estimate_ex_flags_validated():
    lib = _abi.load_library()
    q = t4(SHAPE)
    ha = (ctypes.c_int32 * 1)(0)
    both = _abi.MSA_ESTIMATE_POOL_ONLY | _abi.MSA_ESTIMATE_SELECT_ONLY
    for flags, want in [(16, _abi.MSA_E_FLAGS), (-1, _abi.MSA_E_FLAGS),
                        (both, _abi.MSA_E_FLAGS),
                        (3, _abi.MSA_E_WORKSPACE),
                        (_abi.MSA_ESTIMATE_POOL_ONLY, _abi.MSA_E_WORKSPACE),
                        (_abi.MSA_ESTIMATE_SELECT_ONLY | 3, _abi.MSA_E_WORKSPACE)]:
        st = lib.msa_block_estimate_ex(ctypes.byref(q), ctypes.byref(q), ha, None, 1, 64, 2,
                                       0.088, flags, FAKE, FAKE, FAKE, 100, None)
        assert st == want, flags
    # the message names the flags, not another argument
    assert "flags" in _abi.status_str(_abi.MSA_E_FLAGS)


def test_stage_kv_pool_validated():
    """msa_stage_kv_pool checks the staging arguments and, with block slots,
    the estimator's (fake pointers: nothing is launched)."""
    lib = _abi.load_library()
    q = t4(SHAPE)
    ha = (ctypes.c_int32 * 2)(0, 5)
    need_att = _abi.attention_workspace_bytes(1, 4, 256, 96)
    need_est = _abi.estimate_workspace_bytes(1, 1, 256, 256, 96)

    def call(n_slots=1, heads_arr=ha, est_ws=FAKE, est_b=need_est, ws=FAKE, wsb=need_att, k=q):
        return lib.msa_stage_kv_pool(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k),
                                     heads_arr, n_slots, est_ws, est_b, ws, wsb, None)

    assert call(wsb=need_att - 1) == _abi.MSA_E_WORKSPACE
    assert call(est_b=need_est - 1) == _abi.MSA_E_WORKSPACE
    assert call(est_ws=None) == _abi.MSA_E_WORKSPACE
    assert call(n_slots=2) == _abi.MSA_E_HEADS  # head 5 of 4
    assert call(n_slots=-1) == _abi.MSA_E_HEADS
    assert call(heads_arr=None) == _abi.MSA_E_NULL
    assert call(k=t4([1, 4, 256, 80])) == _abi.MSA_E_HEAD_DIM


def test_one_pass_estimate_needs_caller_workspace():
    """The select pass reads what the pooling pass left in the workspace, so
    the Python wrapper refuses a one-pass call without a large enough one
    (instead of allocating a fresh, unfilled workspace)."""
    import torch

    q = torch.zeros(1, 2, 256, 96, dtype=torch.bfloat16)
    idx = torch.zeros(1, 1, 4, 2, dtype=torch.int32)
    cnt = torch.zeros(1, 1, 4, dtype=torch.int32)
    for phase in (_abi.MSA_ESTIMATE_POOL_ONLY, _abi.MSA_ESTIMATE_SELECT_ONLY):
        with pytest.raises(ValueError, match="workspace"):
            _abi.block_estimate(q, q, [0], [2], 2, 0.088, idx, cnt, flags=phase)
        with pytest.raises(ValueError, match="workspace"):
            _abi.block_estimate(q, q, [0], [2], 2, 0.088, idx, cnt,
                                ws=torch.zeros(16, dtype=torch.uint8), flags=phase)


def test_attention_block_slot_range():
    hd = heads(4, kind=_abi.MSA_KIND_BLOCK, slot=0)
    hd[3].slot = 4
    st = attn(t4(SHAPE), t4(SHAPE), t4(SHAPE), t4(SHAPE), hd, 4, idx=FAKE, cnt=FAKE, slots=4, topk=2)
    assert st == _abi.MSA_E_SLOTS


@pytest.mark.parametrize(
    "kw,expected",
    [
        ({"block": 32}, _abi.MSA_E_BLOCK),
        ({"block": 96}, _abi.MSA_E_BLOCK),
        ({"block": 1000}, _abi.MSA_E_BLOCK),
        ({"block": 0}, _abi.MSA_E_BLOCK),
        ({"block": 128, "topk_max": 3}, _abi.MSA_E_TOPK),  # 256 tokens -> 2 blocks of 128
        ({"topk_max": 0}, _abi.MSA_E_TOPK),
        ({"topk_max": 5}, _abi.MSA_E_TOPK),  # 256 tokens -> 4 blocks
        ({"topk_list": [1, 9]}, _abi.MSA_E_TOPK),
        ({"heads_list": [0, 4]}, _abi.MSA_E_HEADS),
        ({"heads_list": []}, _abi.MSA_E_HEADS),
        ({"scale": -1.0}, _abi.MSA_E_TOPK),
        ({"wsb": 10}, _abi.MSA_E_WORKSPACE),
        ({"idx": None}, _abi.MSA_E_NULL),
    ],
)
def test_estimator_validation(kw, expected):
    args = {"heads_list": [0, 1], "topk_list": [2, 2], "topk_max": 2}
    args.update(kw)
    if "topk_list" in kw or "heads_list" in kw:
        n = len(args["heads_list"])
        if "topk_list" not in kw:
            args["topk_list"] = [2] * n
    hl = args.pop("heads_list")
    tl = args.pop("topk_list")
    tm = args.pop("topk_max")
    assert est(t4(SHAPE), t4(SHAPE), hl, tl, tm, **args) == expected


def dec(q, k, v, o, scale=0.1, ws=FAKE, wsb=1 << 40):
    lib = _abi.load_library()
    return lib.msa_decode_attention(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v),
                                    ctypes.byref(o), scale, ws, wsb, None)


QD, KD = [2, 8, 1, 96], [2, 2, 4096, 96]


@pytest.mark.parametrize(
    "mutate,expected",
    [
        (lambda a: a.__setitem__("q", t4([2, 8, 2, 96])) or a.__setitem__("o", t4([2, 8, 2, 96])), _abi.MSA_E_SEQ),
        (lambda a: a.__setitem__("k", t4([2, 3, 4096, 96])) or a.__setitem__("v", t4([2, 3, 4096, 96])), _abi.MSA_E_RANK),
        (lambda a: a.__setitem__("v", t4([2, 2, 4000, 96])), _abi.MSA_E_RANK),
        (lambda a: a.__setitem__("o", t4([2, 8, 1, 64])), _abi.MSA_E_RANK),
        (lambda a: a.__setitem__("v", t4(KD, _abi.MSA_DTYPE_FP16)), _abi.MSA_E_DTYPE),
        (lambda a: a.__setitem__("o", t4(QD, _abi.MSA_DTYPE_FP16)), _abi.MSA_E_DTYPE),
        (lambda a: a.__setitem__("k", t4(KD, data=FAKE + 8)), _abi.MSA_E_ALIGN),
        (lambda a: a.__setitem__("scale", 0.0), _abi.MSA_E_HEADS),
        (lambda a: a.__setitem__("scale", float("nan")), _abi.MSA_E_HEADS),
        (lambda a: a.__setitem__("k", t4([1, 1, 1 << 20, 128], strides=[0, 0, 2048, 1]))
         or a.__setitem__("q", t4([1, 1, 1, 128])) or a.__setitem__("o", t4([1, 1, 1, 128]))
         or a.__setitem__("v", t4([1, 1, 1 << 20, 128], strides=[0, 0, 2048, 1])), _abi.MSA_E_SEQ),
        (lambda a: a.__setitem__("wsb", 100), _abi.MSA_E_WORKSPACE),
        (lambda a: a.__setitem__("v", t4(KD, data=0)), _abi.MSA_E_NULL),
    ],
)
def test_decode_validation(mutate, expected):
    a = {"q": t4(QD), "k": t4(KD), "v": t4(KD), "o": t4(QD), "scale": 0.1, "wsb": 1 << 40}
    mutate(a)
    assert dec(a["q"], a["k"], a["v"], a["o"], a["scale"], wsb=a["wsb"]) == expected


def test_decode_workspace_sizes():
    # about 2048 split workgroups in all, >= 64 keys each; (D + 2) fp32 per split
    assert _abi.decode_workspace_bytes(1, 32, 65536, 96) == 32 * 64 * 98 * 4
    assert _abi.decode_workspace_bytes(1, 32, 100, 96) == (32 * 2 * 98 * 4 + 255) // 256 * 256
    assert _abi.decode_workspace_bytes(4, 128, 8192, 128) == 512 * 4 * 130 * 4
    assert _abi.decode_workspace_bytes(1, 1, 0, 96) == 0


def rope(q, k, c, s, qo, ko):
    lib = _abi.load_library()
    return lib.msa_rope_qk(*[ctypes.byref(x) for x in (q, k, c, s, qo, ko)], None)


RQ, RK, RC = [2, 8, 300, 96], [2, 2, 300, 96], [1, 1, 300, 96]


@pytest.mark.parametrize(
    "mutate,expected",
    [
        (lambda a: a.__setitem__("k", t4([2, 2, 299, 96])) or a.__setitem__("ko", t4([2, 2, 299, 96])), _abi.MSA_E_RANK),
        (lambda a: a.__setitem__("qo", t4([2, 8, 300, 64])), _abi.MSA_E_RANK),
        (lambda a: a.__setitem__("c", t4([3, 1, 300, 96])) or a.__setitem__("s", t4([3, 1, 300, 96])), _abi.MSA_E_RANK),
        (lambda a: a.__setitem__("c", t4([1, 2, 300, 96])) or a.__setitem__("s", t4([1, 2, 300, 96])), _abi.MSA_E_RANK),
        (lambda a: a.__setitem__("s", t4([1, 1, 300, 64])), _abi.MSA_E_RANK),
        (lambda a: a.__setitem__("c", t4([1, 1, 300, 40])) or a.__setitem__("s", t4([1, 1, 300, 40])), _abi.MSA_E_HEAD_DIM),
        (lambda a: a.__setitem__("c", t4([1, 1, 300, 112])) or a.__setitem__("s", t4([1, 1, 300, 112])), _abi.MSA_E_HEAD_DIM),
        (lambda a: [a.__setitem__(n, t4([2, 8, 300, 36])) for n in ("q", "qo")]
         and [a.__setitem__(n, t4([2, 2, 300, 36])) for n in ("k", "ko")]
         and [a.__setitem__(n, t4([1, 1, 300, 16])) for n in ("c", "s")], _abi.MSA_E_HEAD_DIM),
        (lambda a: a.__setitem__("q", t4(RQ, _abi.MSA_DTYPE_FP16)), _abi.MSA_E_DTYPE),
        (lambda a: [a.__setitem__(n, t4(sh, _abi.MSA_DTYPE_FP32)) for n, sh in
                    (("q", RQ), ("k", RK), ("c", RC), ("s", RC), ("qo", RQ), ("ko", RK))], _abi.MSA_E_DTYPE),
        (lambda a: a.__setitem__("c", t4(RC, data=FAKE + 4)), _abi.MSA_E_ALIGN),
        (lambda a: a.__setitem__("ko", t4(RK, strides=[300 * 96 * 2, 300 * 96, 99, 1])), _abi.MSA_E_ALIGN),
        (lambda a: a.__setitem__("qo", t4(RQ, data=0)), _abi.MSA_E_NULL),
    ],
)
def test_rope_validation(mutate, expected):
    a = {"q": t4(RQ), "k": t4(RK), "c": t4(RC), "s": t4(RC), "qo": t4(RQ), "ko": t4(RK)}
    mutate(a)
    assert rope(a["q"], a["k"], a["c"], a["s"], a["qo"], a["ko"]) == expected


def test_python_ops_refuse_cpu_tensors():
    import torch

    from minference import block_sparse_attention, dense_attention, streaming_forward

    q = torch.randn(1, 2, 128, 96, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        streaming_forward(q, q, q, 64, 128)
    with pytest.raises(RuntimeError, match="GPU only"):
        block_sparse_attention(q, q, q, 2)
    with pytest.raises(RuntimeError, match="GPU only"):
        dense_attention(q, q, q)
    with pytest.raises(AssertionError):
        streaming_forward(q[0], q, q, 64, 128)
    from minference.backend.attention import decode_dense

    with pytest.raises(RuntimeError, match="GPU only"):
        decode_dense(q[:, :, :1], q, q)
    with pytest.raises(NotImplementedError):
        decode_dense(q, q, q)
    from minference.ops.rope import apply_rotary_pos_emb

    cos = torch.zeros(1, 128, 96, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        apply_rotary_pos_emb(q, q, cos, cos)


def test_skip_kind_is_exempt_from_head_checks():
    """MSA_KIND_SKIP heads are left out of a launch: their other fields are
    not checked, and they do not count as causal heads for S_q > S_k (each
    call then fails later, on the deliberately small workspace)."""
    q, kv = t4([1, 4, 512, 96]), t4([1, 4, 256, 96])
    hd = heads(4, kind=_abi.MSA_KIND_FULL)
    hd[1].kind = _abi.MSA_KIND_SKIP
    hd[1].scale = 0.0
    hd[1].slot = 99
    assert attn(q, kv, kv, q, hd, 4, wsb=100) == _abi.MSA_E_WORKSPACE
    hd[2].kind = _abi.MSA_KIND_STREAM
    assert attn(q, kv, kv, q, hd, 4, wsb=100) == _abi.MSA_E_SEQ



def test_head_dim_padding_helpers():
    """Head dims up to 512 run at the next built size (zero padding); the
    scale keeps the reference's rule for the original head_dim;
    vertical_and_slash takes the built sizes up to 128 only."""
    import torch

    from minference.ops import common as C

    assert [C.kernel_head_dim(d) for d in (1, 40, 64, 65, 80, 96, 97, 112, 128, 129, 160, 256,
                                           257, 512)] == \
        [64, 64, 64, 96, 96, 96, 128, 128, 128, 256, 256, 256, 512, 512]
    with pytest.raises(NotImplementedError):
        C.kernel_head_dim(513)
    C.require_kernel_head_dim(256, "x")
    with pytest.raises(NotImplementedError):
        C.require_kernel_head_dim(256, "vertical_and_slash", C.VS_HEAD_DIMS)
    with pytest.raises(NotImplementedError):
        C.require_kernel_head_dim(160, "x")
    # (next allowed of 16/32/64/128/256/512)^-0.5, not of the padded size
    assert C.sparse_scale(24) == 32 ** -0.5 and C.sparse_scale(80) == 128 ** -0.5
    t = torch.arange(2 * 3 * 5 * 40, dtype=torch.float32).reshape(2, 3, 5, 40)
    p = C.pad_head_dim(t, 64)
    assert p.shape == (2, 3, 5, 64) and torch.equal(p[..., :40], t) and not p[..., 40:].any()
    assert C.pad_head_dim(t, 40) is t
    seen = {}

    def fn(q, k, v, r):
        seen["d"] = q.shape[-1]
        r.copy_(q + 1)

    out = C.padded_call(t, t, t, None, fn)
    assert seen["d"] == 64 and out.shape == t.shape and torch.equal(out, t + 1)


def test_float32_inputs_round_to_16_bit():
    """float32 op inputs: fp16 when every finite value fits its range, else
    bf16 (non-finite values ignored by the rule); the decorator hands the op
    the roundings and a float32 output, passes other dtypes through, and
    refuses a non-float32 ``out`` for float32 inputs."""
    import torch

    from minference.ops import common as C

    small = torch.tensor([[1.0, -65504.0, float("inf"), float("nan")]])
    big = torch.tensor([[1.0, 70000.0]])
    assert C.sixteen_bit_dtype([small, small]) == torch.float16
    assert C.sixteen_bit_dtype([small, big]) == torch.bfloat16
    assert C.sixteen_bit_dtype([torch.empty(0)]) == torch.float16

    seen = {}

    @C.accepts_float32(("q", "k"))
    def op(q, k, scale=1.0, *, out=None):
        seen.update(q=q.dtype, k=k.dtype, out=None if out is None else out.dtype, scale=scale)
        return out

    q = torch.ones(1, 2, 3, 4)
    res = op(q, q * 2, 0.5)
    assert seen == {"q": torch.float16, "k": torch.float16, "out": torch.float32, "scale": 0.5}
    assert res.dtype == torch.float32 and res.shape == q.shape
    op(q, q * 1e5)
    assert seen["q"] == torch.bfloat16 and seen["k"] == torch.bfloat16
    seen.clear()
    op(q.bfloat16(), q.bfloat16())
    assert seen["q"] == torch.bfloat16 and seen["out"] is None
    with pytest.raises(ValueError):
        op(q, q, out=torch.empty(q.shape, dtype=torch.bfloat16))

    @C.accepts_float32(("q",), has_out=False)
    def sel(q):
        return q.dtype

    assert sel(q) == torch.float16
