"""Seeded random sweep of layer shapes and pattern mixes on the GPU.

Each case draws batch, head counts (MHA, GQA, MQA), head dim, dtype, S_k
(ragged, down to one key), S_q (full or chunked prefill) and a per-head mix
of stream_llm (random n_init / n_local), block_sparse (random top-k), dense
and, for full prefills, vertical_and_slash heads (random vertical / slash
counts), runs the patched layer's dispatch (run_layer_attention: the
estimators and the attention launches) and checks every row of every head
against the oracle's per-head layer within 2e-3 (fp32 output), plus the
block ids of every block_sparse head bit-exact.
Semantics mirrored: minference/modules/minference_forward.py:398-487 and the
ops it dispatches to (ops/streaming_kernel_npu.py:94-146,
ops/block_sparse_kernel_npu.py:230-348, backend_npu/attention.py:166-255)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O
from msa_data import dtype_tag, make_qkv, np32
from test_gpu_kernels import assert_close_f32, to_dev

pytestmark = pytest.mark.gpu

N_CASES = 40
N_WIDE_CASES = 8  # head dim 256 (no vertical_and_slash heads: built up to 128)


def _draw(i: int):
    rng = np.random.default_rng(20261202 + i)
    D = int(rng.choice([64, 96, 96, 128]))
    if i >= N_CASES:
        D = 256
    B = int(rng.choice([1, 1, 2]))
    Hkv = int(rng.choice([1, 2, 4]))
    H = Hkv * int(rng.choice([1, 2, 3]))
    S_k = int(rng.choice([int(rng.integers(1, 200)), int(rng.integers(200, 1400)),
                          int(rng.integers(1400, 3000))]))
    S_q = S_k if rng.random() < 0.6 else int(rng.integers(1, S_k + 1))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    sink = 8.0 if rng.random() < 0.5 else None
    n_kb = math.ceil(S_k / 64)
    pats = {}
    vs_ok = S_q == S_k and D <= 128
    for h in range(H):
        kind = rng.choice(["stream_llm", "block_sparse", "dense", "vertical_and_slash"],
                          p=[0.3, 0.35, 0.1, 0.25] if vs_ok else [0.4, 0.45, 0.15, 0.0])
        if kind == "vertical_and_slash":
            pats[h] = ["vertical_and_slash", int(rng.integers(1, 1500)), int(rng.integers(1, 3000)),
                       1.0]
        elif kind == "stream_llm":
            pats[h] = ["stream_llm", int(rng.integers(0, 300)), int(rng.integers(1, 2000)), 1.0]
        elif kind == "block_sparse":
            pats[h] = ["block_sparse", min(int(rng.integers(1, 40)), n_kb), 0, 1.0]
        else:
            pats[h] = ["dense", 0, 0, 1.0]
    return B, H, Hkv, S_q, S_k, D, dtype, sink, pats


@pytest.mark.parametrize("i", range(N_CASES + N_WIDE_CASES))
def test_random_layer(gpu_device, i):
    from minference import _abi
    from minference.modules.minference_forward import build_layer_plan, run_layer_attention
    from minference.ops.common import sparse_scale

    B, H, Hkv, S_q, S_k, D, dtype, sink, pats = _draw(i)
    kinds = "".join(pats[h][0][0] for h in range(H))
    print(f"[random] case {i}: B={B} H={H} Hkv={Hkv} S_q={S_q} S_k={S_k} D={D} "
          f"{dtype_tag(dtype)} heads={kinds}", flush=True)
    q, k, v = make_qkv(B, H, S_q, S_k, D, dtype, seed=3000 + i, sink_scale=sink)
    k, v = k[:, :Hkv].contiguous(), v[:, :Hkv].contiguous()
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    plan = build_layer_plan(pats, H, D, S_k)
    out = torch.empty((B, H, S_q, D), dtype=torch.float32, device=gpu_device)
    run_layer_attention(dq, dk, dv, plan, out)

    rep = H // Hkv
    qn = np32(q)
    kr, vr = np.repeat(np32(k), rep, axis=1), np.repeat(np32(v), rep, axis=1)
    ref = np.zeros(q.shape)
    sel = {}
    for h in range(H):
        ty, p1, p2 = pats[h][:3]
        sl = slice(h, h + 1)
        if ty == "vertical_and_slash":
            vi, si = O.vs_estimate(qn[:, sl], kr[:, sl], p1, p2, dtype_tag(dtype))
            ref[:, sl] = O.vertical_slash_from_indices(qn[:, sl], kr[:, sl], vr[:, sl], vi, si)
        else:
            r, s_h = O.layer_attention(qn[:, sl], kr[:, sl], vr[:, sl], [pats[h]], dtype_tag(dtype))
            ref[:, sl] = r
            if 0 in s_h:
                sel[h] = s_h[0]
    assert_close_f32(out, ref, what=f"random case {i}")

    if plan.block_heads:
        ns = len(plan.block_heads)
        n_qb = math.ceil(S_q / 64)
        idx = torch.full((B, ns, n_qb, plan.topk_max), -5, dtype=torch.int32, device=gpu_device)
        cnt = torch.empty((B, ns, n_qb), dtype=torch.int32, device=gpu_device)
        _abi.block_estimate(dq, dk, plan.block_heads, plan.block_topk, plan.topk_max,
                            sparse_scale(D), idx, cnt)
        got_i, got_c = idx.cpu().numpy(), cnt.cpu().numpy()
        for s, h in enumerate(plan.block_heads):
            ridx, rcnt = sel[h]
            tk = plan.block_topk[s]
            assert np.array_equal(got_i[:, s, :, :tk], ridx[:, 0]), f"case {i} head {h}: ids differ"
            want_c = O.attend_count(ridx[:, 0], S_q, S_k)
            assert np.array_equal(got_c[:, s], want_c), f"case {i} head {h}: counts differ"


N_OP_CASES = 24       # head dims up to 128
N_OP_WIDE_CASES = 8   # head dims 130 .. 256 (zero-padded to 256)
N_OP_BLOCK_CASES = 6  # block_sparse_attention with blocks of 128 to 512 tokens


def _draw_op(i: int):
    rng = np.random.default_rng(77000 + i)
    if i < N_OP_CASES:
        D = int(rng.choice([2 * int(rng.integers(4, 65)), 64, 96, 128]))  # even: RoPE'd inputs
    else:
        D = int(rng.choice([2 * int(rng.integers(65, 129)), 256]))
    B = int(rng.choice([1, 2]))
    H = int(rng.integers(1, 5))
    S_k = int(rng.choice([int(rng.integers(1, 300)), int(rng.integers(300, 2500))]))
    S_q = S_k if rng.random() < 0.6 else int(rng.integers(1, S_k + 1))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    op = str(rng.choice(["stream", "block", "dense", "full"]))
    if op == "full":  # dense without the causal mask: any S_q
        S_q = int(rng.integers(1, 2 * S_k + 2))
    n_init, n_local = int(rng.integers(0, 400)), int(rng.integers(1, 3000))
    topk = int(rng.integers(1, 60))
    bs = 64
    if i >= N_OP_CASES + N_OP_WIDE_CASES:
        op, bs = "block", int(rng.choice([128, 192, 256, 320, 512]))
        D = int(rng.choice([64, 80, 96, 128, 256]))
        S_q = min(S_q, S_k)
        topk = int(rng.integers(1, 12))
    return B, H, S_q, S_k, D, dtype, op, n_init, n_local, topk, bs


@pytest.mark.parametrize("i", range(N_OP_CASES + N_OP_WIDE_CASES + N_OP_BLOCK_CASES))
def test_random_op(gpu_device, i):
    """The op-level entry points (streaming_forward, block_sparse_attention
    with blocks of 64 to 512 tokens, dense_attention causal and not) at random
    shapes and head dims up to 256 (zero-padded to the built sizes), fp32
    outputs against the oracle on the
    unpadded inputs (ops/streaming_kernel_npu.py:349-397,
    ops/block_sparse_kernel_npu.py:609-709, backend_npu/attention.py:192-255)."""
    from minference import block_sparse_attention, dense_attention, streaming_forward
    from minference.ops.block_sparse_kernel import select_block_sparse_topk_indices

    B, H, S_q, S_k, D, dtype, op, n_init, n_local, topk, bs = _draw_op(i)
    print(f"[random op] case {i}: {op} B={B} H={H} S_q={S_q} S_k={S_k} D={D} {dtype_tag(dtype)} "
          f"n_init={n_init} n_local={n_local} topk={topk} block={bs}", flush=True)
    q, k, v = make_qkv(B, H, S_q, S_k, D, dtype, seed=5000 + i, sink_scale=8.0,
                       use_rope=S_q <= S_k)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    qn, kn, vn = np32(q), np32(k), np32(v)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    if op == "stream":
        streaming_forward(dq, dk, dv, n_init, n_local, out=out)
        ref = O.streaming_attention(qn, kn, vn, n_init, n_local)
    elif op == "block":
        n_kb = math.ceil(S_k / bs)
        ids = select_block_sparse_topk_indices(dq, dk, topk, bs).cpu().numpy()
        ref_ids, _ = O.select_block_sparse_topk_indices(qn, kn, min(topk, n_kb), dtype_tag(dtype),
                                                        block=bs)
        assert np.array_equal(ids, ref_ids), f"case {i}: ids differ"
        block_sparse_attention(dq, dk, dv, topk, bs, out=out)
        ref = O.block_sparse_from_indices(qn, kn, vn, ref_ids, block=bs)
    elif op == "dense":
        dense_attention(dq, dk, dv, out=out)
        ref = O.dense_causal(qn, kn, vn)
    else:
        dense_attention(dq, dk, dv, causal=False, out=out)
        ref = O.dense_causal(qn, kn, vn, causal=False)
    assert_close_f32(out, ref, what=f"random op case {i}")


@pytest.mark.parametrize("i", range(16))
def test_random_decode(gpu_device, i):
    """decode_dense (one query row against the whole cache; split-K partials
    and their merge) at random cache lengths, GQA groups and head dims up to
    256 (backend_npu/attention.py:274-314)."""
    from minference.backend.attention import decode_dense

    rng = np.random.default_rng(91000 + i)
    if i < 12:
        D = int(rng.choice([2 * int(rng.integers(4, 65)), 64, 96, 128]))  # even: RoPE'd inputs
    else:
        D = int(rng.choice([2 * int(rng.integers(65, 129)), 256]))
    B = int(rng.choice([1, 2, 3]))
    Hkv = int(rng.choice([1, 2, 4]))
    H = Hkv * int(rng.choice([1, 2, 4]))
    S = int(rng.choice([int(rng.integers(1, 200)), int(rng.integers(200, 20000))]))
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    print(f"[random decode] case {i}: B={B} H={H} Hkv={Hkv} S={S} D={D} {dtype_tag(dtype)}",
          flush=True)
    q, _, _ = make_qkv(B, H, 1, S, D, dtype, seed=6000 + i)
    _, k, v = make_qkv(B, Hkv, S, S, D, dtype, seed=6100 + i, sink_scale=8.0)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    decode_dense(dq, dk, dv, out=out)
    rep = H // Hkv
    ref = O.dense_causal(np32(q), np.repeat(np32(k), rep, axis=1), np.repeat(np32(v), rep, axis=1))
    assert_close_f32(out, ref, what=f"random decode case {i}")


@pytest.mark.parametrize("i", range(12))
def test_random_rope(gpu_device, i):
    """msa_rope_qk at random shapes (head dims multiples of 8, rotary widths
    multiples of 16 up to the head dim, GQA, per-batch or broadcast tables,
    random table halves): bit-exact with HF's eager apply_rotary_pos_emb on
    the same GPU (looked up at minference/modules/minference_forward.py:205-212)."""
    from minference.ops.rope import apply_rotary_pos_emb, rope_supported
    from test_rope import hf_rope, rope_tables

    rng = np.random.default_rng(88000 + i)
    D = 8 * int(rng.integers(2, 17))
    rot = 16 * int(rng.integers(1, D // 16 + 1))
    B = int(rng.choice([1, 2]))
    Hkv = int(rng.choice([1, 2, 4]))
    H = Hkv * int(rng.choice([1, 2, 4]))
    S = int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(64, 3000))]))
    dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float16
    tb = B if rng.random() < 0.5 else 1
    rnd = bool(rng.random() < 0.5)
    print(f"[random rope] case {i}: B={B} H={H} Hkv={Hkv} S={S} D={D} rot={rot} "
          f"{dtype_tag(dtype)} tables={tb} random={rnd}", flush=True)
    g = torch.Generator().manual_seed(8800 + i)
    q = (torch.randn(B, H, S, D, generator=g) * 3).to(dtype)
    k = (torch.randn(B, Hkv, S, D, generator=g) * 3).to(dtype)
    cos, sin = rope_tables(tb, S, rot, dtype, offset=int(rng.integers(0, 100000)),
                           random_halves=rnd, seed=i)
    dq, dk, dc, ds = to_dev(gpu_device, q, k, cos, sin)
    assert rope_supported(dq, dk, dc, ds)
    gq, gk = apply_rotary_pos_emb(dq, dk, dc, ds)
    rq, rk = hf_rope(dq, dk, dc, ds)
    torch.cuda.synchronize()
    assert torch.equal(gq, rq) and torch.equal(gk, rk), f"random rope case {i}"
