"""Parity of the exact launch the benchmark times (its default workload).

bench.py's headline step: S = 65536, 32 heads x 96, bf16, 16 stream_llm(128,
4096) + 16 block_sparse(top-100) heads assigned by the seed-0 shuffle, Q/K/V
from the bench's own generator (RoPE, K rows 0-3 x8), launched by the
bench's own schedule (launch_block_layer: estimator pooling, selection beside
the K/V staging, one attention launch with the plan's kind-interleaved,
cost-balanced item order; the fp32 output by a second launch).  Checked here:
  * block ids of all 16 block heads bit-exact with the oracle;
  * 8 rows in every query block of every head (8192 x 32 rows, at
    offsets that move with the block and the head) plus the tile
    boundaries, the sink edge, the band start and the last rows, within
    2e-3 of the oracle's fp64 rows, in fp32 output and in the bf16 output
    the bench writes (plus one bf16 rounding);
  * every row of every head through a constant-V launch (the output of a
    softmax-weighted mean of a constant is that constant).
Reference semantics: minference/ops/streaming_kernel_npu.py:94-146,
minference/ops/block_sparse_kernel_npu.py:230-263, 325-348."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O
import row_sampling as RS

pytestmark = pytest.mark.gpu

TOL = 2e-3
S, H, D = 65536, 32, 96


def _rows(n_init, n_local):
    base = {0, 1, 63, 64, 65, 127, 128, 129, 191, 192, n_init - 1, n_init, n_local - 1, n_local,
            n_local + 1, n_local + n_init - 1, n_local + n_init, n_local + 63, n_local + 64,
            8191, 8192, S // 2 - 1, S // 2, S - 65, S - 64, S - 63, S - 2, S - 1}
    return sorted(r for r in base if 0 <= r < S)


def test_headline_launch_matches_oracle(gpu_device):
    import bench
    from minference import _abi
    from minference.modules.minference_forward import build_layer_plan, launch_block_layer
    from minference.ops.common import sparse_scale

    print("[headline] building the bench's layer", flush=True)
    pats, counts = bench.layer_patterns("headline", H, seed=0)
    assert counts == (16, 16, 0)
    plan = build_layer_plan(pats, H, D, S)
    q, k, v = bench.make_inputs(S, H, D, 0, gpu_device)
    n_qb = math.ceil(S / 64)
    n_slots = len(plan.block_heads)
    idx = torch.empty((1, n_slots, n_qb, plan.topk_max), dtype=torch.int32, device=gpu_device)
    cnt = torch.empty((1, n_slots, n_qb), dtype=torch.int32, device=gpu_device)
    ws = _abi.workspace(_abi.attention_workspace_bytes(1, H, S, D), gpu_device)
    est_ws = _abi.workspace(_abi.estimate_workspace_bytes(1, n_slots, S, S, D), gpu_device)
    out16 = torch.empty_like(q)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    launch_block_layer(q, k, v, plan, out16, idx, cnt, ws, est_ws)
    _abi.layer_attention(q, k, v, out32, plan.heads, idx=idx, cnt=cnt, idx_slots=n_slots,
                         topk_max=plan.topk_max, ws=ws, staged=True)
    torch.cuda.synchronize()

    print("[headline] oracle block ids", flush=True)
    qn = q.float().cpu().numpy()[0]
    kn = k.float().cpu().numpy()[0]
    vn = v.float().cpu().numpy()[0]
    bh = list(plan.block_heads)
    ridx, rcnt = O.select_block_sparse_topk_indices(qn[bh], kn[bh], 100, "bf16", sparse_scale(D))
    got_idx = idx.cpu().numpy()[0]
    assert np.array_equal(cnt.cpu().numpy()[0], rcnt)
    assert np.array_equal(got_idx, ridx), f"{(got_idx != ridx).sum()} block ids differ"

    print("[headline] 8 rows per query block of every head", flush=True)
    o32 = out32.cpu().numpy()[0]
    o16 = out16.float().cpu().numpy()[0]
    sc = sparse_scale(D)

    def check(h):
        kind, p1, p2, slot, _ = plan.heads[h]
        assert kind in (_abi.MSA_KIND_STREAM, _abi.MSA_KIND_BLOCK)
        rows = RS.block_rows(S, h, per_block=8, extra=_rows(128, 4096))
        ids = ridx[slot] if kind == _abi.MSA_KIND_BLOCK else None
        cn = rcnt[slot] if kind == _abi.MSA_KIND_BLOCK else None
        ref = RS.head_rows_reference(qn[h], kn[h], vn[h], rows, kind, p1, p2, sc, ids, cn)
        err = np.abs(o32[h, rows] - ref)
        bad16 = np.abs(o16[h, rows] - ref) > TOL + np.abs(ref) * 2.0 ** -8
        return h, kind, rows.size, float(err.max()), int((err >= TOL).sum()), int(bad16.sum())

    res = RS.map_heads(check, range(H), tag="[headline]")
    n_rows = sum(r[2] for r in res)
    worst = max(r[3] for r in res)
    print(f"[headline] {n_rows} rows, worst error {worst:.3e}", flush=True)
    for h, kind, n, err, n_bad, n_bad16 in res:
        assert n_bad == 0 and n_bad16 == 0, (h, kind, n, err, n_bad, n_bad16)

    print("[headline] constant V, every row", flush=True)
    c = (torch.arange(H, device=gpu_device, dtype=torch.float32) * 0.25 + 0.5)
    vc = c.view(1, H, 1, 1).expand(1, H, S, D).to(torch.bfloat16).contiguous()
    _abi.stage_kv(k, vc, ws)
    _abi.layer_attention(q, k, vc, out32, plan.heads, idx=idx, cnt=cnt, idx_slots=n_slots,
                         topk_max=plan.topk_max, ws=ws, staged=True)
    dev = (out32 - c.view(1, H, 1, 1)).abs().amax(dim=(0, 2, 3)) / c
    assert float(dev.max()) < 1e-3, dev.cpu().tolist()
