"""The layer schedule (launch_block_layer), the estimator's one-pass flags and
MSA_KIND_SKIP heads on the GPU.

A layer with block_sparse heads runs the K/V staging with the estimator's
pooling pass in the same launch, then the selection pass, then one attention
launch of all heads, all on one stream.  The passes compute what one estimator call computes,
and the attention launch is the one msa_layer_attention makes, so the ids
and the output must equal those of the plain calls bit for bit; their
correctness against the oracle is what the other GPU tests check.
Semantics mirrored: minference/modules/minference_forward.py:398-487 (the
reference's per-kind dispatch of one layer)."""

from __future__ import annotations

import math

import pytest
import torch

from msa_data import make_qkv
from test_gpu_kernels import to_dev

pytestmark = pytest.mark.gpu


def _layer(gpu_device, H, Hkv, S, kinds, seed, big_v_kv=None):
    from minference.modules.minference_forward import build_layer_plan

    q, _, _ = make_qkv(1, H, S, S, 96, torch.bfloat16, seed=seed, sink_scale=8.0)
    _, k, v = make_qkv(1, Hkv, S, S, 96, torch.bfloat16, seed=seed + 1, sink_scale=8.0)
    if big_v_kv is not None:
        v = v.clone()
        v[0, big_v_kv, 5::97, 3] = 2.0e5  # beyond fp16: this kv head stages scaled
    rec = {"stream_llm": ["stream_llm", 64, 256, 1.0], "block_sparse": ["block_sparse", 6, 0, 1.0],
           "dense": ["dense", 0, 0, 1.0]}
    pats = {h: list(rec[kd]) for h, kd in enumerate(kinds)}
    plan = build_layer_plan(pats, H, 96, S)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    return plan, dq, dk, dv


def _single_launch(plan, q, k, v, idx, cnt, out):
    from minference import _abi

    _abi.layer_attention(q, k, v, out, plan.heads, idx=idx, cnt=cnt,
                         idx_slots=len(plan.block_heads), topk_max=plan.topk_max)


@pytest.mark.parametrize("case", ["gqa_mixed", "mha_mixed", "block_only"])
def test_layer_schedule_matches_plain_calls(gpu_device, case):
    """launch_block_layer (staging + pooling in one launch, then the
    selection, one stream) == msa_block_estimate + msa_layer_attention,
    bit for bit, fp32 and bf16 outputs, twice in a row.  gqa_mixed: kv heads
    shared by block and stream heads, one kv head holding V beyond the fp16
    range."""
    from minference import _abi
    from minference.modules.minference_forward import launch_block_layer
    from minference.ops.common import sparse_scale

    print(f"[schedule] {case}", flush=True)
    S = 1500
    if case == "gqa_mixed":
        # kv 0: stream+block, kv 1: block only (big V), kv 2: dense+stream, kv 3: block+dense
        kinds = ["stream_llm", "block_sparse", "block_sparse", "block_sparse",
                 "dense", "stream_llm", "block_sparse", "dense"]
        plan, q, k, v = _layer(gpu_device, 8, 4, S, kinds, seed=3, big_v_kv=1)
    elif case == "mha_mixed":
        kinds = ["block_sparse", "stream_llm", "dense", "block_sparse", "stream_llm", "block_sparse"]
        plan, q, k, v = _layer(gpu_device, 6, 6, S, kinds, seed=4)
    else:
        plan, q, k, v = _layer(gpu_device, 4, 2, S, ["block_sparse"] * 4, seed=5)
    n_qb = math.ceil(S / 64)
    ns = len(plan.block_heads)
    idx = torch.empty((1, ns, n_qb, plan.topk_max), dtype=torch.int32, device=gpu_device)
    cnt = torch.empty((1, ns, n_qb), dtype=torch.int32, device=gpu_device)
    idx2, cnt2 = torch.full_like(idx, -5), torch.full_like(cnt, -5)
    _abi.block_estimate(q, k, plan.block_heads, plan.block_topk, plan.topk_max,
                        sparse_scale(96), idx2, cnt2)
    ws = _abi.workspace(_abi.attention_workspace_bytes(1, k.shape[1], S, 96), gpu_device)
    est_ws = _abi.workspace(_abi.estimate_workspace_bytes(1, ns, S, S, 96), gpu_device)
    for dt in (torch.float32, torch.bfloat16):
        ref = torch.empty(q.shape, dtype=dt, device=gpu_device)
        _single_launch(plan, q, k, v, idx2, cnt2, ref)
        for rep in range(2):
            out = torch.full(q.shape, float("nan"), dtype=dt, device=gpu_device)
            idx.fill_(-5)
            cnt.fill_(-5)
            launch_block_layer(q, k, v, plan, out, idx, cnt, ws, est_ws)
            torch.cuda.synchronize()
            assert torch.equal(idx, idx2) and torch.equal(cnt, cnt2)
            assert torch.equal(out, ref), (case, dt, rep, float((out.float() - ref.float()).abs().max()))


def test_skip_heads_are_not_written(gpu_device):
    """Heads marked MSA_KIND_SKIP keep their output rows untouched; the other
    heads equal the all-heads launch."""
    from minference import _abi

    print("[schedule] skip heads", flush=True)
    kinds = ["stream_llm", "dense", "stream_llm", "dense"]
    plan, q, k, v = _layer(gpu_device, 4, 4, 700, kinds, seed=6)
    ref = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    _abi.layer_attention(q, k, v, ref, plan.heads)
    skip = [0, 3]
    heads = [(_abi.MSA_KIND_SKIP, 0, 0, -1, 1.0) if h in skip else hd
             for h, hd in enumerate(plan.heads)]
    out = torch.full(q.shape, -7.0, dtype=torch.float32, device=gpu_device)
    _abi.layer_attention(q, k, v, out, heads)
    torch.cuda.synchronize()
    for h in range(4):
        if h in skip:
            assert bool((out[:, h] == -7.0).all()), h
        else:
            assert torch.equal(out[:, h], ref[:, h]), h


def test_run_layer_attention_uses_split_schedule(gpu_device):
    """The patched forward's layer call on a mixed layer equals the single
    launch (it goes through launch_block_layer)."""
    from minference import _abi
    from minference.modules.minference_forward import run_layer_attention

    kinds = ["block_sparse", "stream_llm", "block_sparse", "dense"]
    plan, q, k, v = _layer(gpu_device, 4, 4, 1024, kinds, seed=8)
    out = torch.empty_like(q)
    run_layer_attention(q, k, v, plan, out)
    n_qb = 16
    idx = torch.empty((1, 2, n_qb, plan.topk_max), dtype=torch.int32, device=gpu_device)
    cnt = torch.empty((1, 2, n_qb), dtype=torch.int32, device=gpu_device)
    from minference.ops.common import sparse_scale

    _abi.block_estimate(q, k, plan.block_heads, plan.block_topk, plan.topk_max,
                        sparse_scale(96), idx, cnt)
    ref = torch.empty_like(q)
    _single_launch(plan, q, k, v, idx, cnt, ref)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("block", [64, 192])
@pytest.mark.parametrize("flags", [0, 3])
def test_estimator_passes_match_one_call(gpu_device, flags, block):
    """MSA_ESTIMATE_POOL_ONLY then MSA_ESTIMATE_SELECT_ONLY (on another
    stream, ordered by an event) == one msa_block_estimate_ex call, ids and
    counts bit for bit, with and without the forced first / diagonal blocks,
    at 64- and 192-token blocks; the pooling pass leaves idx and cnt
    untouched."""
    from minference import _abi
    from minference.modules.minference_forward import _side_stream
    from minference.ops.common import sparse_scale

    print(f"[schedule] estimator passes flags={flags} block={block}", flush=True)
    S = 2000
    kinds = ["block_sparse", "stream_llm", "block_sparse", "block_sparse"]
    plan, q, k, v = _layer(gpu_device, 4, 2, S, kinds, seed=11)
    n_qb = math.ceil(S / block)
    ns = len(plan.block_heads)
    topk = [3, 6, 5]
    idx = torch.empty((1, ns, n_qb, 6), dtype=torch.int32, device=gpu_device)
    cnt = torch.empty((1, ns, n_qb), dtype=torch.int32, device=gpu_device)
    ref_idx, ref_cnt = torch.full_like(idx, -5), torch.full_like(cnt, -5)
    sc = sparse_scale(96)
    _abi.block_estimate(q, k, plan.block_heads, topk, 6, sc, ref_idx, ref_cnt, flags=flags,
                        block=block)
    ws = _abi.workspace(_abi.estimate_workspace_bytes(1, ns, S, S, 96), gpu_device)
    idx.fill_(-5)
    cnt.fill_(-5)
    _abi.block_estimate(q, k, plan.block_heads, topk, 6, sc, idx, cnt, ws,
                        flags=flags | _abi.MSA_ESTIMATE_POOL_ONLY, block=block)
    torch.cuda.synchronize()
    assert bool((idx == -5).all()) and bool((cnt == -5).all())
    side = _side_stream(q.device)
    side.wait_stream(torch.cuda.current_stream(q.device))
    with torch.cuda.stream(side):
        _abi.block_estimate(q, k, plan.block_heads, topk, 6, sc, idx, cnt, ws,
                            flags=flags | _abi.MSA_ESTIMATE_SELECT_ONLY, block=block)
    torch.cuda.current_stream(q.device).wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(idx, ref_idx) and torch.equal(cnt, ref_cnt)
