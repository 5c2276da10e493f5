"""vertical_and_slash on the GPU through the C ABI, against the oracle.

Attention for given (v_idx, s_idx): the tile-list build, the gathered
vertical tiles and the VS instantiation of the attention kernel, alone and in
a mixed layer next to stream / block / dense heads."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from msa_data import dtype_tag, make_qkv, np32
from test_gpu_kernels import assert_close_f32, assert_close_lowp, to_dev

pytestmark = pytest.mark.gpu


def _vs_lists(S, n_v, n_s, B, H, seed, kind="mixed"):
    """Index sets in the reference tests' style (tests/test_vertical_slash_kernel.py:
    47-76): 30 sink columns + random columns, 100 local slashes + random far
    ones; plus special shapes."""
    g = np.random.default_rng(seed)
    v = np.zeros((B, H, n_v), np.int64)
    s = np.zeros((B, H, n_s), np.int64)
    for b in range(B):
        for h in range(H):
            if kind == "mixed":
                vv = np.concatenate([np.arange(min(30, S)), g.integers(0, S, n_v)])
                ss = np.concatenate([np.arange(min(100, S)), g.integers(0, S, n_s)])
            elif kind == "vertical":    # no slash reaches any row
                vv = g.integers(0, S, n_v)
                ss = np.full(n_s, S + 64)
            elif kind == "slash":       # verticals all inside slash windows (column 0)
                vv = np.zeros(n_v, np.int64)
                ss = g.integers(0, S, n_s)
            elif kind == "messy":       # repeats, out of range, negative slashes
                vv = g.integers(-50, S + 50, n_v)
                ss = g.integers(-200, S + 200, n_s)
            elif kind == "clustered":   # verticals in a few far tiles
                base = g.integers(0, max(1, S - 64), 3)
                vv = (base[:, None] + g.integers(0, 64, (3, n_v // 3 + 1))).ravel()
                ss = np.concatenate([np.arange(min(16, S)), g.integers(0, S, n_s)])
            v[b, h] = np.sort(vv[:n_v])
            s[b, h] = np.sort(ss[:n_s])[::-1]
    return v, s


VS_CASES = [
    # (B, H, S, D, n_v, n_s, dtype, kind)
    (1, 2, 64, 96, 40, 60, torch.bfloat16, "mixed"),
    (1, 2, 300, 96, 60, 120, torch.bfloat16, "mixed"),
    (2, 2, 1000, 96, 100, 200, torch.bfloat16, "mixed"),
    (1, 3, 4096 + 17, 96, 500, 300, torch.bfloat16, "mixed"),
    (1, 2, 2048, 64, 300, 150, torch.float16, "mixed"),
    (1, 2, 2048, 128, 300, 150, torch.bfloat16, "clustered"),
    (1, 2, 1500, 96, 200, 50, torch.bfloat16, "vertical"),
    (1, 2, 1500, 96, 40, 400, torch.bfloat16, "slash"),
    (1, 2, 1200, 96, 300, 300, torch.bfloat16, "messy"),
]


@pytest.mark.parametrize("case", VS_CASES, ids=[f"{c[:6]}{dtype_tag(c[6])}-{c[7]}" for c in VS_CASES])
def test_vs_attention_vs_oracle(gpu_device, case):
    from minference.ops.vertical_slash_kernel import vertical_slash_sparse_attention

    B, H, S, D, n_v, n_s, dtype, kind = case
    print(f"[vs] case {case}", flush=True)
    q, k, v = make_qkv(B, H, S, S, D, dtype, seed=S + n_v, sink_scale=8.0)
    vi, si = _vs_lists(S, n_v, n_s, B, H, seed=S, kind=kind)
    ref = O.vertical_slash_from_indices(np32(q), np32(k), np32(v), vi, si)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    vertical_slash_sparse_attention(dq, dk, dv, torch.from_numpy(vi), torch.from_numpy(si),
                                    out=out32)
    assert_close_f32(out32, ref, what=f"vs {case}")
    out = vertical_slash_sparse_attention(dq, dk, dv, torch.from_numpy(vi), torch.from_numpy(si))
    assert out.dtype == dtype
    assert_close_lowp(out, ref, what=f"vs lowp {case}")


def test_vs_full_coverage_equals_dense(gpu_device):
    """tests/test_vertical_slash_kernel.py:289-303 on the GPU."""
    from minference.ops.vertical_slash_kernel import vertical_slash_sparse_attention

    B, H, S, D = 1, 2, 777, 96
    q, k, v = make_qkv(B, H, S, S, D, torch.bfloat16, seed=4)
    vi = torch.arange(S).expand(B, H, S)
    si = torch.arange(S - 1, -1, -1).expand(B, H, S)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    vertical_slash_sparse_attention(dq, dk, dv, vi, si, out=out32)
    ref = O.dense_causal(np32(q), np32(k), np32(v), scale=O.sparse_scale(D))
    assert_close_f32(out32, ref, what="vs full coverage")


@pytest.mark.parametrize("H_kv", [8, 2])
def test_vs_in_mixed_layer(gpu_device, H_kv):
    """VS heads next to stream / block / dense heads in one
    msa_layer_attention_ex call (two attention launches), GQA included."""
    from minference import _abi
    from minference.ops.block_sparse_kernel import select_block_sparse_topk_indices
    from minference.ops.vertical_slash_kernel import canonical_vertical_lists

    B, H, S, D = 1, 8, 2000, 96
    q, _, _ = make_qkv(B, H, S, S, D, torch.bfloat16, seed=21)
    _, k, v = make_qkv(B, H_kv, S, S, D, torch.bfloat16, seed=22, sink_scale=8.0)
    kinds = ["vs", "stream", "vs", "block", "dense", "vs", "vs", "block"]
    vs_heads = [h for h in range(H) if kinds[h] == "vs"]
    blk_heads = [h for h in range(H) if kinds[h] == "block"]
    vi, si = _vs_lists(S, 150, 120, B, len(vs_heads), seed=5)
    sc = O.sparse_scale(D)
    heads = []
    for h in range(H):
        if kinds[h] == "vs":
            heads.append((_abi.MSA_KIND_VS, 0, 0, vs_heads.index(h), sc))
        elif kinds[h] == "stream":
            heads.append((_abi.MSA_KIND_STREAM, 64, 512, -1, sc))
        elif kinds[h] == "block":
            heads.append((_abi.MSA_KIND_BLOCK, 6, 0, blk_heads.index(h), sc))
        else:
            heads.append((_abi.MSA_KIND_DENSE, 0, 0, -1, O.dense_scale(D)))
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    rep = H // H_kv
    kn = np.repeat(np32(k), rep, 1)
    vn = np.repeat(np32(v), rep, 1)
    qn = np32(q)
    # block ids from the GPU estimator (bit-exact with the oracle elsewhere)
    kr = dk.repeat_interleave(rep, 1)
    idx, cnt = select_block_sparse_topk_indices(dq[:, blk_heads], kr[:, blk_heads], 6,
                                                return_counts=True)
    idx32 = idx.to(torch.int32).contiguous()
    v_ids, v_cnt = canonical_vertical_lists(torch.from_numpy(vi).to(gpu_device), S)
    s_t = torch.from_numpy(si).to(device=gpu_device, dtype=torch.int32).contiguous()
    s_cnt = torch.full((B, len(vs_heads)), si.shape[-1], dtype=torch.int32, device=gpu_device)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    _abi.layer_attention(dq, dk, dv, out, heads, idx=idx32, cnt=cnt.to(torch.int32).contiguous(),
                         idx_slots=len(blk_heads), topk_max=6, vs=(v_ids, v_cnt, s_t, s_cnt))
    ref = np.zeros(q.shape)
    idx_np = idx.cpu().numpy()
    for h in range(H):
        sl = slice(h, h + 1)
        if kinds[h] == "vs":
            j = vs_heads.index(h)
            ref[:, sl] = O.vertical_slash_from_indices(qn[:, sl], kn[:, sl], vn[:, sl],
                                                       vi[:, j:j + 1], si[:, j:j + 1], scale=sc)
        elif kinds[h] == "stream":
            ref[:, sl] = O.streaming_attention(qn[:, sl], kn[:, sl], vn[:, sl], 64, 512, scale=sc)
        elif kinds[h] == "block":
            j = blk_heads.index(h)
            ref[:, sl] = O.block_sparse_from_indices(qn[:, sl], kn[:, sl], vn[:, sl],
                                                     idx_np[:, j:j + 1], scale=sc)
        else:
            ref[:, sl] = O.dense_causal(qn[:, sl], kn[:, sl], vn[:, sl])
    assert_close_f32(out, ref, what=f"mixed layer with VS heads (H_kv={H_kv})")


# ---------------------------------------------------------------------------
# estimator: bit-exact indices
# ---------------------------------------------------------------------------
EST_CASES = [
    # (B, H, H_kv, S, D, vertical_size, slash_size, dtype)
    (1, 2, 2, 40, 96, 30, 50, torch.bfloat16),          # S < 64 rows, every index taken
    (1, 2, 2, 100, 96, 30, 50, torch.bfloat16),
    (1, 2, 2, 1000, 96, 100, 300, torch.bfloat16),
    (2, 2, 2, 4096 + 17, 96, 1000, 6096, torch.bfloat16),
    (1, 4, 2, 2048, 64, 200, 80, torch.bfloat16),       # fewer slashes than forced diagonals, GQA
    (1, 2, 2, 3000, 128, 500, 700, torch.float16),
]


@pytest.mark.parametrize("case", EST_CASES, ids=[f"{c[:7]}{dtype_tag(c[7])}" for c in EST_CASES])
def test_vs_estimator_bit_exact(gpu_device, case):
    from minference.ops.vertical_slash_kernel import vertical_and_slash_estimate

    B, H, Hkv, S, D, vsz, ssz, dtype = case
    print(f"[vs-est] case {case}", flush=True)
    q, _, _ = make_qkv(B, H, S, S, D, dtype, seed=S + vsz)
    _, k, _ = make_qkv(B, Hkv, S, S, D, dtype, seed=S + ssz, sink_scale=8.0)
    v_idx, s_idx = vertical_and_slash_estimate(*to_dev(gpu_device, q, k), vsz, ssz)
    rv, rs = O.vs_estimate(np32(q), np32(k), vsz, ssz, dtype_tag(dtype))
    gv, gs = v_idx.cpu().numpy(), s_idx.cpu().numpy()
    assert gv.shape == rv.shape and gs.shape == rs.shape
    assert np.array_equal(gv, rv), f"{(gv != rv).sum()} vertical ids differ"
    assert np.array_equal(gs, rs), f"{(gs != rs).sum()} slash ids differ"


@pytest.mark.parametrize("S,vsz,ssz", [(2048, 300, 500), (4096 + 17, 1000, 6096)])
def test_vs_estimate_and_attention_vs_oracle(gpu_device, S, vsz, ssz):
    """The reference's _vertical_and_slash_kernel end to end
    (minference_forward.py:140-167): estimator, then the sparse attention."""
    from minference.ops.vertical_slash_kernel import vertical_and_slash_attention

    B, H, D = 1, 2, 96
    q, k, v = make_qkv(B, H, S, S, D, torch.bfloat16, seed=S, sink_scale=8.0)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    vertical_and_slash_attention(dq, dk, dv, vsz, ssz, out=out32)
    vi, si = O.vs_estimate(np32(q), np32(k), vsz, ssz, "bf16")
    ref = O.vertical_slash_from_indices(np32(q), np32(k), np32(v), vi, si)
    assert_close_f32(out32, ref, what=f"vs pipeline S={S}")
