"""V values outside the fp16 range, and non-finite V, on the GPU.

The PV product runs on the fp16 MFMA with V staged once per layer as fp16.
bf16 V can exceed fp16's finite range (65504): such a head is staged times an
exact power of two and its output scaled back, so the result still matches
the reference's fp32 arithmetic (minference/ops/streaming_kernel_npu.py:
138-143, minference/ops/block_sparse_kernel_npu.py:342-348).  Inf and NaN in V
are never turned into finite values: every row that attends to such a key
returns a non-finite output in that dimension."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from msa_data import make_qkv, np32
from test_gpu_kernels import to_dev

pytestmark = pytest.mark.gpu

REL = 2e-3


def _big_v(v: torch.Tensor, heads, seed=0, mag=1.0e5, n=40):
    """Plant +-mag (bf16) at n random (key, dim) places of each listed head."""
    g = torch.Generator().manual_seed(seed)
    v = v.clone()
    S, D = v.shape[2], v.shape[3]
    for h in heads:
        keys = torch.randint(0, S, (n,), generator=g)
        dims = torch.randint(0, D, (n,), generator=g)
        sign = torch.randint(0, 2, (n,), generator=g).float() * 2 - 1
        v[0, h, keys, dims] = (sign * mag).to(v.dtype)
    return v


def _assert_rel(got: torch.Tensor, ref: np.ndarray, ref_abs: np.ndarray, what: str):
    """|got - ref| <= 2e-3 * max(1, sum_j p_j |v_j|) elementwise (the error of
    a weighted mean scales with the weighted mean of |v|)."""
    g = got.detach().float().cpu().numpy().astype(np.float64)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    bound = REL * np.maximum(1.0, ref_abs)
    worst = (np.abs(g - ref) / bound).max()
    assert worst <= 1.0, f"{what}: error {worst:.2f} x the bound"


@pytest.mark.parametrize("D,mag", [(96, 1.0e5), (96, 1.0e6), (256, 1.0e5), (512, 1.0e6)])
def test_mixed_layer_v_beyond_fp16(gpu_device, D, mag):
    """stream / block / dense heads of one launch, bf16 V holding +-mag
    entries in two of the four heads (the other two stay in range); the V
    exponents are 1 and 5.  (P reaches the PV product as fp16 with full
    relative precision down to 2^-21 of the row's largest weight; a key
    weighted below that contributes an error of at most 2^-32 |V| per key,
    so the bound here holds for |V| up to about 1e6.)"""
    from minference import _abi
    from minference.ops.block_sparse_kernel import select_block_sparse_topk_indices

    print(f"[vrange] mixed layer D={D} mag={mag}", flush=True)
    B, H, S = 1, 4, 1500
    q, k, v = make_qkv(B, H, S, S, D, torch.bfloat16, seed=17, sink_scale=8.0)
    v = _big_v(v, heads=(0, 2), mag=mag)
    assert v.float().abs().max() > 65504
    sc = O.sparse_scale(D)
    heads = [(_abi.MSA_KIND_STREAM, 64, 512, -1, sc), (_abi.MSA_KIND_BLOCK, 5, 0, 0, sc),
             (_abi.MSA_KIND_DENSE, 0, 0, -1, O.dense_scale(D)), (_abi.MSA_KIND_BLOCK, 5, 0, 1, sc)]
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    idx, cnt = select_block_sparse_topk_indices(dq[:, [1, 3]], dk[:, [1, 3]], 5, return_counts=True)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    _abi.layer_attention(dq, dk, dv, out, heads, idx=idx.to(torch.int32).contiguous(),
                         cnt=cnt.to(torch.int32).contiguous(), idx_slots=2, topk_max=5)
    qn, kn, vn = np32(q), np32(k), np32(v)
    ridx, _ = O.select_block_sparse_topk_indices(qn[:, [1, 3]], kn[:, [1, 3]], 5, "bf16")
    ref = np.zeros(q.shape)
    ref_abs = np.zeros(q.shape)
    for vv, dst in ((vn, ref), (np.abs(vn), ref_abs)):
        dst[:, 0:1] = O.streaming_attention(qn[:, 0:1], kn[:, 0:1], vv[:, 0:1], 64, 512)
        dst[:, 1:2] = O.block_sparse_from_indices(qn[:, 1:2], kn[:, 1:2], vv[:, 1:2], ridx[:, 0:1])
        dst[:, 2:3] = O.dense_causal(qn[:, 2:3], kn[:, 2:3], vv[:, 2:3])
        dst[:, 3:4] = O.block_sparse_from_indices(qn[:, 3:4], kn[:, 3:4], vv[:, 3:4], ridx[:, 1:2])
    _assert_rel(out, ref, ref_abs, f"mixed layer mag={mag}")
    # the bf16 output of the same call path (one more rounding)
    from minference import streaming_forward

    o16 = streaming_forward(dq[:, :1], dk[:, :1], dv[:, :1], 64, 512)
    g = o16.float().cpu().numpy()
    assert np.isfinite(g).all()
    assert (np.abs(g - ref[:, :1]) <= REL * np.maximum(1.0, ref_abs[:, :1])
            + np.abs(ref[:, :1]) * 2.0 ** -8).all()


def test_vertical_slash_v_beyond_fp16(gpu_device):
    """The gathered vertical columns of a vertical_and_slash head use the same
    V scale as the head's staged tiles."""
    from minference.ops.vertical_slash_kernel import vertical_slash_sparse_attention
    from test_gpu_vs import _vs_lists

    B, H, S, D = 1, 2, 2000, 96
    q, k, v = make_qkv(B, H, S, S, D, torch.bfloat16, seed=9, sink_scale=8.0)
    vi, si = _vs_lists(S, 300, 150, B, H, seed=3, kind="mixed")
    v = v.clone()
    v[0, :, vi[0, 0, 40:60], 3] = 2.0e5  # big values on gathered vertical columns
    v = _big_v(v, heads=(1,), mag=1.0e5)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    vertical_slash_sparse_attention(dq, dk, dv, torch.from_numpy(vi), torch.from_numpy(si), out=out)
    qn, kn, vn = np32(q), np32(k), np32(v)
    ref = O.vertical_slash_from_indices(qn, kn, vn, vi, si)
    ref_abs = O.vertical_slash_from_indices(qn, kn, np.abs(vn), vi, si)
    _assert_rel(out, ref, ref_abs, "vertical_and_slash")


@pytest.mark.parametrize("D", [96, 256, 512])
def test_nan_and_inf_in_v_propagate(gpu_device, D):
    """A NaN (Inf) at V[key, dim] makes that dim non-finite in every row that
    attends to the key; rows whose tiles never include the key stay exact, and
    no other dimension is touched."""
    from minference import streaming_forward

    print(f"[vrange] nan/inf propagation D={D}", flush=True)
    B, H, S = 1, 2, 1024
    q, k, v = make_qkv(B, H, S, S, D, torch.bfloat16, seed=5)
    n_init, n_local = 64, 256
    kn_, dn_ = 300, 5    # NaN key / dim (head 0)
    ki_, di_ = 700, 7    # +Inf key / dim (head 1)
    v = v.clone()
    v[0, 0, kn_, dn_] = float("nan")
    v[0, 1, ki_, di_] = float("inf")
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    streaming_forward(dq, dk, dv, n_init, n_local, out=out)
    got = out.cpu().numpy()
    clean = np32(v).copy()
    clean[0, 0, kn_, dn_] = 0.0
    clean[0, 1, ki_, di_] = 0.0
    ref = O.streaming_attention(np32(q), np32(k), clean, n_init, n_local)
    rows = np.arange(S)
    for h, key, dim in ((0, kn_, dn_), (1, ki_, di_)):
        sees = (rows >= key) & (rows - n_local < key)  # band rows; key is past the sink
        assert not np.isfinite(got[0, h, sees, dim]).any(), f"head {h}: finite output"
        other = np.ones(D, bool)
        other[dim] = False
        assert np.abs(got[0, h][:, other] - ref[0, h][:, other]).max() < 2e-3
        # rows of query blocks whose tile lists never reach the key's tile
        far = (rows // 64 < key // 64) | (((rows // 64) * 64 - n_local + 1) // 64 > key // 64)
        assert np.isfinite(got[0, h, far, dim]).all()
        assert np.abs(got[0, h, far, dim] - ref[0, h, far, dim]).max() < 2e-3
