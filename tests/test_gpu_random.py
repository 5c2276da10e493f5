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


def _draw(i: int):
    rng = np.random.default_rng(20261202 + i)
    D = int(rng.choice([64, 96, 96, 128]))
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
    vs_ok = S_q == S_k
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


@pytest.mark.parametrize("i", range(N_CASES))
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
