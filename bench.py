#!/usr/bin/env python3
"""Sparse prefill attention benchmark: one Phi-3-mini layer on one MI355X.

A step = the whole sparse attention of one layer, all heads, inputs resident
in HBM, launched as the patched forward launches it (launch_block_layer), in
order on one stream: the K/V staging together with the block estimator's
pooling pass (one launch), the estimator's selection pass (block top-k for
the block_sparse heads), then one attention launch of all heads.  QKV projection, RoPE and o_proj are outside
the step (the reference's per-layer attention, BASELINE.json metric).

Default workload ("headline"): S = 65536, 32 heads x 96, bf16, every head
sparse, 16 stream_llm(n_init 128, n_local 4096) + 16 block_sparse(top-100)
heads (seeded head assignment).  Q, K, V ~ N(0,1) from a seeded generator,
RoPE theta 1e4 on Q and K, K rows 0-3 scaled 8x (attention sinks).

Printed JSON line: value = algorithmic TFLOP/s of the whole step; roofline =
the attention kernel alone (the sum of its launches' durations, HIP events on
the launch stream) against the bf16 MFMA peak; dense = same-GPU dense attention on the same tensors
(PyTorch SDPA flash and this build's dense kind); cpu_baseline = the
reference's CPU path (its torch ops, restated in oracle/cpu_reference.py) for
BASELINE configs 1 (stream_llm) and 2 (block_sparse) timed on the host cores; decode = one decode step against the layer's K/V cache;
rope = the fused RoPE kernel on the layer's q and k against HF's eager one.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "minference-npu_amd"), os.path.join(ROOT, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA (no sparsity)
PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E
BLOCK = 64

# workload -> profile summary holding the calibrated HBM traffic of the attention kernel
TRAFFIC_PROFILE = {"headline": "attn_kernel_headline64k_traffic.txt",
                   "cfg2_block16k": "attn_kernel_cfg2_block16k_traffic.txt",
                   "cfg3_stream64k": "attn_kernel_cfg3_stream64k_traffic.txt"}

WORKLOADS = {
    # name: (S, n_stream, n_block, n_dense, n_init, n_local, topk)
    "headline": (65536, 16, 16, 0, 128, 4096, 100),
    "cfg2_block16k": (16384, 0, 32, 0, 128, 4096, 100),
    "cfg3_stream64k": (65536, 32, 0, 0, 128, 4096, 100),
    "vs64k": (65536, 0, 0, 0, 0, 0, 0),  # VS_MIX below
    # full-model prefill (BASELINE configs 4 and 5): (S, mix) in MODEL_MIX
    "cfg4_prefill32k": (32768, 0, 0, 0, 0, 0, 0),
    "cfg5_prefill128k": (131072, 0, 0, 0, 0, 0, 0),
}

# Selector option per single-layer workload: BASELINE config 2 states "with
# the diagonal and first block always included" (MSA_SELECT_FORCE_FIRST |
# MSA_SELECT_FORCE_DIAG, inside the top-k); the others use the reference's
# plain top-k.
SELECT_FORCE = {"cfg2_block16k": (True, True)}

# Per-head pattern mixes of the full-prefill workloads over all 1024 heads,
# drawn by configs.patterns.mixed_config from the bench seed.
MODEL_MIX = {
    "cfg4_prefill32k": [(0.3, ["stream_llm", 128, 4096]), (0.6, ["block_sparse", 100, 0]),
                        (0.1, ["dense", 0, 0])],
    "cfg5_prefill128k": [(0.5, ["stream_llm", 128, 8192]), (0.5, ["block_sparse", 160, 0])],
}

# The reference's original Phi-3 pattern (1024 heads: vertical_and_slash
# (3500,100) x378, (1000,6096) x277, (100,750) x184, (500,700) x92,
# (30,800) x50, stream_llm (100,800) x43) scaled to one layer of 32 heads.
VS_MIX = [
    (12, ["vertical_and_slash", 3500, 100, 1.0]),
    (9, ["vertical_and_slash", 1000, 6096, 1.0]),
    (6, ["vertical_and_slash", 100, 750, 1.0]),
    (3, ["vertical_and_slash", 500, 700, 1.0]),
    (1, ["vertical_and_slash", 30, 800, 1.0]),
    (1, ["stream_llm", 100, 800, 1.0]),
]


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="headline")
    ap.add_argument("--heads", type=int, default=32)
    ap.add_argument("--dim", type=int, default=96)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-dense", action="store_true", help="skip the same-GPU dense baselines")
    ap.add_argument("--skip-kind", choices=("stream", "block"), default=None,
                    help="profiling aid (not a benchmark line): the attention launch leaves the "
                         "heads of this kind out (MSA_KIND_SKIP), to count one kind's traffic")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode measurement")
    ap.add_argument("--no-rope", action="store_true", help="skip the RoPE measurement")
    ap.add_argument("--cpu-block-heads", type=int, default=2,
                    help="heads of BASELINE config 2 timed on the CPU per repeat (scaled to 32)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (5 launches) to calibrate the "
                         "FETCH_SIZE / WRITE_SIZE counters, then exit")
    return ap.parse_args()


def stream_pairs(s, n_init, n_local):
    import numpy as np

    i = np.arange(s, dtype=np.int64)
    lo = np.maximum(0, i - n_local + 1)
    return int(((i - lo + 1) + np.minimum(n_init, lo)).sum())


def block_tiles(s, topk):
    nb = -(-s // BLOCK)
    k = min(topk, nb)
    return sum(min(k, b + 1) for b in range(nb))


def layer_patterns(workload, H, seed):
    """Per-head pattern records of a single-layer workload: the workload's
    stream / block / dense counts scaled to H heads, assigned to heads by a
    seeded shuffle.  Returns ({head: record}, (n_stream, n_block, n_dense))."""
    import random

    S, n_stream, n_block, n_dense, n_init, n_local, topk = WORKLOADS[workload]
    scale_h = H / (n_stream + n_block + n_dense)
    n_stream, n_block = int(round(n_stream * scale_h)), int(round(n_block * scale_h))
    n_dense = H - n_stream - n_block
    kinds = (["stream_llm"] * n_stream + ["block_sparse"] * n_block + ["dense"] * n_dense)
    random.Random(seed).shuffle(kinds)
    rec = {"stream_llm": ["stream_llm", n_init, n_local, 1.0],
           "block_sparse": ["block_sparse", topk, 0, 1.0],
           "dense": ["dense", 0, 0, 1.0]}
    return {h: list(rec[kd]) for h, kd in enumerate(kinds)}, (n_stream, n_block, n_dense)


def make_inputs(S, H, D, seed, device):
    import torch

    from msa_data import rope

    g = torch.Generator(device=device).manual_seed(seed)
    out = []
    for name in ("q", "k", "v"):
        x = torch.randn(1, H, S, D, generator=g, device=device, dtype=torch.float32)
        if name != "v":
            # RoPE by 4096-row slabs to bound the fp32 temporaries
            for s0 in range(0, S, 4096):
                x[:, :, s0:s0 + 4096] = rope(x[:, :, s0:s0 + 4096], offset=s0)
        if name == "k":
            x[:, :, :4] *= 8.0
        out.append(x.to(torch.bfloat16))
        del x
    return out


def profiled_traffic(workload):
    """HBM bytes of the attention kernel per step (its launches of the layer)
    measured by two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE; calibrated
    on a device copy), from profiles/."""
    name = TRAFFIC_PROFILE.get(workload)
    if not name:
        return None
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for ln in f:
                if ln.startswith("attn_kernel traffic_bytes_per_step:"):
                    return int(ln.split(":")[1])
    except OSError:
        pass
    return None


def cpu_info():
    """CPU model, physical cores of the host, CPUs this process may run on,
    and the threads torch uses."""
    import torch

    model, cores = platform.processor() or "unknown", set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                key, _, val = ln.partition(":")
                key, val = key.strip(), val.strip()
                if key == "model name":
                    model = val
                elif key == "physical id":
                    phys = val
                elif key == "core id":
                    core = val
                elif not key and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
        if phys is not None:
            cores.add((phys, core))
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"cpu_model": model, "physical_cores": len(cores) or None,
            "logical_cpus": os.cpu_count(), "usable_cpus": usable,
            "threads": torch.get_num_threads()}


def _time_cpu(fn, repeats=3):
    fn()  # warmup 1
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return times


def cpu_baseline(block_heads_sample):
    """The reference's CPU path timed on the host (warmup 1, 3 repeats, as
    benchmarks/probe_block_sparse_heads.py:18-31), through the torch-CPU fp32
    restatement in oracle/cpu_reference.py (the reference's own ops at its
    padded D = 128):
      stream_llm, B=1, 32 heads, S=4096, D=96, fp32,
        n_init 64, n_local 1024, all 32 heads per repeat;
      block_sparse top-100 at S=16384, bf16 inputs, one
        head at a time (the as-written [1,32,S,S] fp32 logits are 34 GB);
        ``block_heads_sample`` heads per repeat, scaled to 32 heads.
    value / unit are config 1's algorithmic TFLOP/s."""
    import torch

    from msa_data import make_qkv
    from oracle import cpu_reference as R

    info = cpu_info()
    S, D, n_init, n_local = 4096, 96, 64, 1024
    q, k, v = make_qkv(1, 32, S, S, D, torch.float32, seed=0)
    with torch.no_grad():
        t1 = _time_cpu(lambda: R.streaming_reference(q, k, v, n_init, n_local))
    per1 = sum(t1) / len(t1)
    flop1 = 32 * stream_pairs(S, n_init, n_local) * 4 * D
    del q, k, v

    S2, topk, nh = 16384, 100, max(1, int(block_heads_sample))
    q, k, v = make_qkv(1, nh, S2, S2, D, torch.bfloat16, seed=2, sink_scale=8.0)
    with torch.no_grad():
        t2 = _time_cpu(lambda: R.block_sparse_reference(q, k, v, topk))
    scale2 = 32 / nh
    per2 = sum(t2) / len(t2) * scale2
    flop2 = 32 * block_tiles(S2, topk) * 4 * BLOCK * BLOCK * D
    del q, k, v
    return {
        "value": round(flop1 / per1 / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": info["threads"],
        "kind": "port",
        "sample": ("BASELINE config 1 (stream_llm S=4096 n_init=64 n_local=1024, 32 heads, fp32) "
                   "through a torch-CPU fp32 restatement of the reference CPU path "
                   "(_streaming_pytorch_ref after the D 96->128 pad: chunked full-row logits, "
                   "masked softmax), warmup 1 + 3 repeats of the whole layer"),
        "ms_per_layer": round(per1 * 1e3, 2),
        "ms_min_max": [round(min(t1) * 1e3, 2), round(max(t1) * 1e3, 2)],
        "block_cfg2": {
            "value": round(flop2 / per2 / 1e12, 6), "unit": "TFLOP/s",
            "ms_per_layer": round(per2 * 1e3, 1),
            "ms_min_max": [round(min(t2) * scale2 * 1e3, 1), round(max(t2) * scale2 * 1e3, 1)],
            "sample": (f"BASELINE config 2 (block_sparse top-100, S=16384, bf16) through the "
                       f"torch-CPU restatement of _block_sparse_pytorch_ref (selector, token mask, "
                       f"fp32 masked softmax over S x S, D padded to 128), one head at a time; "
                       f"{nh} of 32 heads x 3 repeats, scaled to 32 heads"),
        },
        **info,
    }


def main():
    args = parse_args()
    if args.calibrate_copy:
        import torch

        n = args.calibrate_copy * (1 << 20) // 2
        src = torch.ones(n, dtype=torch.bfloat16, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_mib": args.calibrate_copy, "launches": 5}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path (heads would shard across GPUs with no communication inside "
              "attention).", file=sys.stderr)
        sys.exit(1)

    import torch

    from minference import _abi
    from minference.modules.minference_forward import build_layer_plan, launch_block_layer
    from minference.ops.common import sparse_scale

    dev = torch.device("cuda:0")
    if args.workload == "vs64k":
        return vs_bench(args, dev)
    if args.workload in MODEL_MIX:
        return model_bench(args, dev)
    S, n_stream, n_block, n_dense, n_init, n_local, topk = WORKLOADS[args.workload]
    H, D = args.heads, args.dim
    pats, (n_stream, n_block, n_dense) = layer_patterns(args.workload, H, args.seed)
    plan = build_layer_plan(pats, H, D, S)
    if args.skip_kind:
        import dataclasses

        skip = _abi.MSA_KIND_STREAM if args.skip_kind == "stream" else _abi.MSA_KIND_BLOCK
        plan = dataclasses.replace(plan, heads=tuple(
            (_abi.MSA_KIND_SKIP,) + tuple(hd[1:]) if hd[0] == skip else hd for hd in plan.heads))
        n_stream, n_block = (0, n_block) if args.skip_kind == "stream" else (n_stream, 0)

    q, k, v = make_inputs(S, H, D, args.seed, dev)
    out = torch.empty_like(q)
    n_qb = math.ceil(S / BLOCK)
    n_slots = len(plan.block_heads)
    idx = torch.empty((1, max(n_slots, 1), n_qb, max(plan.topk_max, 1)), dtype=torch.int32, device=dev)
    cnt = torch.empty((1, max(n_slots, 1), n_qb), dtype=torch.int32, device=dev)
    ws_est = _abi.workspace(_abi.estimate_workspace_bytes(1, max(n_slots, 1), S, S, D), dev)
    ws_att = _abi.workspace(_abi.attention_workspace_bytes(1, H, S, D), dev)
    s_sparse = sparse_scale(D)
    stream = torch.cuda.current_stream(dev)

    force_first, force_diag = SELECT_FORCE.get(args.workload, (False, False))
    sel_flags = ((_abi.MSA_SELECT_FORCE_FIRST if force_first else 0)
                 | (_abi.MSA_SELECT_FORCE_DIAG if force_diag else 0))

    names = ("start", "est0", "est1", "stage0", "stage1", "attn0", "attn0_end")
    ev = [{n: torch.cuda.Event(enable_timing=True) for n in names} for _ in range(args.steps)]
    if not n_slots:
        idx = cnt = None

    def step(e=None):
        # the product's schedule (launch_block_layer): staging + pooling, the
        # selection, then one attention launch of all heads
        if n_slots:
            launch_block_layer(q, k, v, plan, out, idx, cnt, ws_att, ws_est, sel_flags,
                               mark=(lambda n, st: e[n].record(st)) if e else None)
            return
        if e:
            e["start"].record(stream)
            e["stage0"].record(stream)
        _abi.stage_kv(k, v, ws_att)
        if e:
            e["stage1"].record(stream)
            e["attn0"].record(stream)
        _abi.layer_attention(q, k, v, out, plan.heads, ws=ws_att, staged=True)
        if e:
            e["attn0_end"].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    # the per-launch breakdown: K more steps with events at the phase
    # boundaries (outside the timed loop: each timing event adds a little)
    for i in range(args.steps):
        step(ev[i])
    torch.cuda.synchronize()

    def avg(a, b):
        return sum(e[a].elapsed_time(e[b]) for e in ev) / args.steps

    t_est = avg("est0", "est1") if n_slots else 0.0
    # the estimator's own time: both passes as msa_block_estimate runs them
    # (in the step the pooling pass is part of the staging launch)
    t_est_alone = 0.0
    if n_slots:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for rep_i in range(args.warmup + args.steps):
            if rep_i == args.warmup:
                e0.record(stream)
            _abi.block_estimate(q, k, plan.block_heads, plan.block_topk, plan.topk_max,
                                s_sparse, idx, cnt, ws_est, flags=sel_flags)
        e1.record(stream)
        torch.cuda.synchronize()
        t_est_alone = e0.elapsed_time(e1) / args.steps
    t_stage = avg("stage0", "stage1")
    t_attn = avg("attn0", "attn0_end")
    t_pre = avg("start", "attn0")

    flop_stream = n_stream * stream_pairs(S, n_init, n_local) * 4 * D
    flop_block = n_block * block_tiles(S, topk) * 4 * BLOCK * BLOCK * D
    flop_dense_heads = n_dense * (S * (S + 1) // 2) * 4 * D
    flop = flop_stream + flop_block + flop_dense_heads
    achieved_attn = flop / (t_attn * 1e-3) / 1e12
    value = flop / (ms_step * 1e-3) / 1e12
    est_bytes = 2 * n_slots * S * D * 2 + n_slots * n_qb * (plan.topk_max + 1) * 4

    result = {
        "metric": "sparse prefill attn ms/layer + effective TFLOP/s (% MFMA peak) vs dense, Phi-3 64K",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) Q/K/V, RoPE, K rows 0-3 x8)",
        "config": {
            "workload": args.workload,
            "model": "Phi-3-mini layer attention (32 heads x 96)",
            "seq_len": S,
            "heads": H,
            "head_dim": D,
            "mix": {"stream_llm(%d,%d)" % (n_init, n_local): n_stream,
                    "block_sparse(top-%d)" % topk: n_block, "dense": n_dense},
            "selector": ("top-%d, first and diagonal blocks forced" % topk if sel_flags
                         else "top-%d (reference selector)" % topk),
            "global_batch": 1,
            "parallelism": "single GPU",
            **({"skip_kind": args.skip_kind} if args.skip_kind else {}),
        },
        "ms_per_layer": round(ms_step, 4),
        "pct_mfma_peak": round(100 * value / PEAK_BF16_TFLOPS, 2),
        "algorithmic_flop": flop,
        "kernels_ms": ({"stage_kv_pool": round(t_stage, 4), "select": round(t_est, 4),
                        "attention": round(t_attn, 4)} if n_slots else
                       {"stage_kv": round(t_stage, 4), "attention": round(t_attn, 4)}),
        "schedule": ("K/V staging + block pooling (one launch); block selection; one attention "
                     "launch; one stream" if n_slots else "staging; one attention launch"),
        "ms_before_first_attention": round(t_pre, 4),
        "estimator_alone": ({"ms": round(t_est_alone, 4),
                             "gbps": round(est_bytes / (t_est_alone * 1e-3) / 1e9, 1)}
                            if n_slots else None),
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved_attn, 3),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved_attn / PEAK_BF16_TFLOPS, 4),
            "traffic": profiled_traffic(args.workload),
            "kernel": "msa::attn_kernel<Bf16,false,96>",
        },
    }

    if not args.no_decode:
        result["decode"] = decode_bench(k, v, S, H, D, args.seed)
    if not args.no_rope:
        result["rope"] = rope_bench(S, H, D, args.seed)
    if not args.no_dense:
        result["dense"] = dense_baselines(q, k, v, S, H, D, ms_step)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args.cpu_block_heads)
    print(json.dumps(result), flush=True)


def vs_tiles(v_idx, s_idx, S):
    """Key tiles the attention kernel walks for one vertical_and_slash head:
    per query block, the tiles a slash window meets (plus the diagonal tile
    when a vertical column lies in it) and the 64-column groups of gathered
    vertical columns (the tile-list rule of vs_build_kernel)."""
    import numpy as np

    nb = -(-S // BLOCK)
    bq = np.arange(nb)
    end = BLOCK * (bq + 1)
    cov = np.zeros((nb, nb), dtype=bool)
    for s in np.asarray(s_idx).tolist():
        ok = s < end
        hi = np.minimum(np.maximum(end - s, BLOCK), S)
        lo = np.maximum(hi - BLOCK, 0)
        hc = np.minimum(hi, np.minimum(end, S))
        ok &= lo < hc
        rows = bq[ok]
        cov[rows, lo[ok] // BLOCK] = True
        cov[rows, (hc[ok] - 1) // BLOCK] = True
    cov &= bq[None, :] <= bq[:, None]
    cols = np.asarray(v_idx)
    ctile = cols // BLOCK
    total = int(cov.sum())
    for b in range(nb):
        in_diag = (ctile == b).any()
        total += int(in_diag and not cov[b, b])
        gath = (cols < BLOCK * b) & ~cov[b, np.minimum(ctile, nb - 1)]
        if gath.any():
            total += len(np.unique(np.nonzero(gath)[0] // BLOCK))
    return total


def _side_stream(dev):
    from minference.modules.minference_forward import _side_stream as side

    return side(dev)


def phi3_mini_128k(dev, n_layers=32):
    """Random-init Phi-3-mini-128k-shaped model in bf16 on ``dev``: 32 layers,
    hidden 3072, 32 heads x 96, MLP 8192, vocab 32064, LongRoPE tables (the
    checkpoint's factor lists are not available offline; their values do not
    change the work)."""
    import torch
    from transformers import Phi3Config, Phi3ForCausalLM

    cfg = Phi3Config(vocab_size=32064, hidden_size=3072, intermediate_size=8192,
                     num_hidden_layers=n_layers, num_attention_heads=32, num_key_value_heads=32,
                     max_position_embeddings=131072, original_max_position_embeddings=4096,
                     rope_scaling={"type": "longrope", "short_factor": [1.0] * 48,
                                   "long_factor": [4.0] * 48},
                     pad_token_id=32000, bos_token_id=1, eos_token_id=32000)
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            torch.manual_seed(0)
            model = Phi3ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(old)
    return model.eval()


def model_bench(args, dev):
    """--workload cfg4_prefill32k / cfg5_prefill128k: full prefill of the
    random-init Phi-3-mini-128k-shaped model through the patched forward
    (MInference with a seeded per-head pattern file over all 1024 heads),
    use_cache=True, last-token logits.  value = TTFT (ms).  The patched
    forward's attention launches (estimators + staging + attention of each
    layer) and RoPE launches are bracketed by HIP events, which gives the
    attention fraction of prefill time; the unpatched model (PyTorch SDPA) on
    the same ids is the dense baseline."""
    import tempfile

    import torch

    from minference import MInference
    from minference.configs import patterns as PAT
    from minference.modules import minference_forward as MF

    S = WORKLOADS[args.workload][0]
    mix = [(f, PAT.record(*rec)) for f, rec in MODEL_MIX[args.workload]]
    model = phi3_mini_128k(dev)
    ids = torch.randint(3, 32000, (1, S), device=dev,
                        generator=torch.Generator(device=dev).manual_seed(args.seed))
    stream = torch.cuda.current_stream(dev)

    def ttft(m, reps):
        times = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            with torch.no_grad():
                m(input_ids=ids, use_cache=True, logits_to_keep=1)
            torch.cuda.synchronize()
            times.append((time.perf_counter() - t0) * 1e3)
        return times

    dense = None
    if not args.no_dense:
        ttft(model, 1)
        dense = ttft(model, 1)[0]
        torch.cuda.empty_cache()

    cfg = PAT.mixed_config(mix, seed=args.seed)
    with tempfile.NamedTemporaryFile("w", suffix=".json", delete=False) as f:
        path = f.name
    PAT.write(path, cfg)
    model = MInference(attn_type="minference", config_path=path)(model)
    events = {"attention": [], "rope": []}
    real_attn, real_rope = MF.run_layer_attention, MF._apply_rope

    def timed(key, fn):
        def wrapper(*a, **kw):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            r = fn(*a, **kw)
            e1.record(stream)
            events[key].append((e0, e1))
            return r
        return wrapper

    MF.run_layer_attention = timed("attention", real_attn)
    MF._apply_rope = timed("rope", real_rope)
    try:
        for _ in range(args.warmup):
            ttft(model, 1)
        for v in events.values():
            v.clear()
        runs = ttft(model, max(1, args.steps))
        torch.cuda.synchronize()
        per_run = {k: sum(a.elapsed_time(b) for a, b in v) / len(runs) for k, v in events.items()}
    finally:
        MF.run_layer_attention, MF._apply_rope = real_attn, real_rope
        os.unlink(path)
    t = sum(runs) / len(runs)
    kinds = PAT.validate_config(cfg).kind_counts()
    result = {
        "metric": "Phi-3-mini-128k-shaped full prefill TTFT (patched, all heads per the mix)",
        "value": round(t, 2), "unit": "ms", "n_gpus": 1, "steps": len(runs), "warmup": args.warmup,
        "ms_per_step": round(t, 2), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights, random token ids)",
        "config": {"workload": args.workload, "model": "Phi-3-mini-128k shape, 32 layers",
                   "seq_len": S, "heads": 32, "head_dim": 96, "mix": kinds,
                   "global_batch": 1, "parallelism": "single GPU"},
        "ttft_runs_ms": [round(x, 2) for x in runs],
        "attention_ms": round(per_run["attention"], 2),
        "attention_fraction": round(per_run["attention"] / t, 4),
        "rope_ms": round(per_run["rope"], 2),
        "dense_sdpa_ttft_ms": round(dense, 2) if dense is not None else None,
        "speedup_vs_dense_ttft": round(dense / t, 2) if dense is not None else None,
    }
    print(json.dumps(result), flush=True)


def vs_bench(args, dev):
    """--workload vs64k: one layer of the reference's original Phi-3 pattern mix
    at 64K (VS_MIX): vertical_and_slash estimator + K/V staging + attention
    (tile-list build, vertical gather, VS kernel, and the stream head's
    kernel)."""
    import random

    import torch

    from minference import _abi
    from minference.modules.minference_forward import build_layer_plan, _vs_lists

    S, H, D = 65536, args.heads, args.dim
    kinds = [rec for n, rec in VS_MIX for _ in range(n)]
    random.Random(args.seed).shuffle(kinds)
    plan = build_layer_plan({h: kinds[h] for h in range(H)}, H, D, S)
    q, k, v = make_inputs(S, H, D, args.seed, dev)
    out = torch.empty_like(q)
    ws_att = _abi.workspace(_abi.attention_workspace_bytes(1, H, S, D), dev)
    nv = max(c[0] for c in plan.vs_counts)
    vs_ws = _abi.workspace(_abi.vs_workspace_bytes(1, len(plan.vs_heads), S, nv, D), dev)
    stream = torch.cuda.current_stream(dev)
    lists = [None]

    side = _side_stream(dev)

    def step(e=None):
        if e:
            e[0].record(stream)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            if e:
                e[4].record(side)
            _abi.stage_kv(k, v, ws_att)
            if e:
                e[5].record(side)
        lists[0] = _vs_lists(q, k, plan)
        if e:
            e[1].record(stream)
        stream.wait_stream(side)
        if e:
            e[2].record(stream)
        _abi.layer_attention(q, k, v, out, plan.heads, ws=ws_att, staged=True, vs=lists[0],
                             vs_ws=vs_ws)
        if e:
            e[3].record(stream)

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(6)] for _ in range(args.steps)]
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    for i in range(args.steps):  # the breakdown, outside the timed loop
        step(ev[i])
    torch.cuda.synchronize()
    t_est = sum(e[0].elapsed_time(e[1]) for e in ev) / args.steps
    t_stage = sum(e[4].elapsed_time(e[5]) for e in ev) / args.steps
    t_attn = sum(e[2].elapsed_time(e[3]) for e in ev) / args.steps

    v_idx, v_cnt, s_idx, s_cnt = (t.cpu() for t in lists[0])
    tiles = 0
    for j, h in enumerate(plan.vs_heads):
        tiles += vs_tiles(v_idx[0, j, :int(v_cnt[0, j])].numpy(),
                          s_idx[0, j, :int(s_cnt[0, j])].numpy(), S)
    # the tile-list builder's own totals, read from the workspace (layout of
    # vs_layout in msa_abi.hip: the per-wave lists, then (unmasked, total)
    # per row and wave; wave w walks the 16-key chunk w of its tiles)
    n_kb = -(-S // BLOCK)
    nv_pad = -(-max(nv, 1) // BLOCK) * BLOCK
    cap = n_kb + nv_pad // BLOCK
    n_rows = len(plan.vs_heads) * n_kb
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    cnt_off = up(n_rows * 4 * cap * 4)
    counts = vs_ws[cnt_off:cnt_off + n_rows * 32].view(torch.int32).view(n_rows, 4, 2).cpu()
    chunks = int(counts[:, :, 1].sum())
    n_stream = sum(1 for hd in plan.heads if hd[0] == _abi.MSA_KIND_STREAM)
    flop_vs = chunks * 4 * BLOCK * (BLOCK // 4) * D
    flop_stream = n_stream * stream_pairs(S, 100, 800) * 4 * D
    flop = flop_vs + flop_stream
    dense_flop = H * (S * (S + 1) // 2) * 4 * D
    result = {
        "metric": "vertical_and_slash prefill attn ms/layer, Phi-3 64K (original pattern mix)",
        "value": round(flop / (ms_step * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) Q/K/V, RoPE, K rows 0-3 x8)",
        "config": {
            "workload": "vs64k", "seq_len": S, "heads": H, "head_dim": D,
            "mix": {f"{r[0]}({r[1]},{r[2]})": n for n, r in VS_MIX},
            "global_batch": 1, "parallelism": "single GPU",
        },
        "ms_per_layer": round(ms_step, 4),
        "kernels_ms": {"vs_estimate": round(t_est, 4), "stage_kv": round(t_stage, 4),
                       "lists_gather_attention": round(t_attn, 4)},
        "vs_tiles": tiles,
        "vs_chunks_builder": chunks,
        "vs_chunks_unmasked": int(counts[:, :, 0].sum()),
        "vs_tile_density": round(tiles / (len(plan.vs_heads) * block_tiles(S, 1 << 30)), 4),
        "executed_flop": flop,
        "attention_tflops": round(flop / (t_attn * 1e-3) / 1e12, 3),
        "dense_equivalent_tflops": round(dense_flop / (ms_step * 1e-3) / 1e12, 3),
    }
    if not args.no_dense:
        result["dense"] = dense_baselines(q, k, v, S, H, D, ms_step)
    print(json.dumps(result), flush=True)


def decode_bench(k, v, S, H, D, seed, reps=20):
    """One decode step of the layer (msa_decode_attention: q [1,H,1,D] against
    the whole K/V cache of S keys), timed with HIP events on the launch
    stream.  K and V (4*D bytes per key and head) are read once per step and
    exceed the on-die cache at the headline length, so the step is bound by
    HBM."""
    import torch

    from minference import _abi
    from minference.ops.common import dense_scale

    g = torch.Generator(device=k.device).manual_seed(seed + 7)
    q1 = torch.randn((1, H, 1, D), generator=g, device=k.device).to(k.dtype)
    out = torch.empty_like(q1)
    ws = _abi.workspace(_abi.decode_workspace_bytes(1, H, S, D), k.device)
    sc = dense_scale(D)
    stream = torch.cuda.current_stream(k.device)
    for _ in range(3):
        _abi.decode_attention(q1, k, v, out, sc, ws)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * reps)]
    torch.cuda.synchronize()
    for i in range(reps):
        ev[2 * i].record(stream)
        _abi.decode_attention(q1, k, v, out, sc, ws)
        ev[2 * i + 1].record(stream)
    torch.cuda.synchronize()
    us = sum(ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(reps)) / reps * 1e3
    nbytes = 2 * H * S * D * k.element_size()
    gbps = nbytes / (us * 1e-6) / 1e9
    return {"s_k": S, "heads": H, "us_per_layer": round(us, 2), "kv_bytes": nbytes,
            "hbm_gbps": round(gbps, 1), "frac_hbm_peak": round(gbps / PEAK_HBM_GBPS, 4),
            "kernels": "msa::decode_kernel + msa::decode_combine_kernel"}


def rope_bench(S, H, D, seed, reps=10):
    """RoPE of one layer's q and k (msa_rope_qk, in place on the views of a
    fused qkv projection output, as the patched forward runs it) against the
    eager HF apply_rotary_pos_emb on the same views, HIP events on the launch
    stream.  Algorithmic bytes: q and k read and written once, plus the
    cos/sin tables."""
    import torch

    from minference.ops.rope import apply_rotary_pos_emb
    from transformers.models.phi3.modeling_phi3 import apply_rotary_pos_emb as hf_rope

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(seed + 11)
    qkv = torch.randn((1, S, 3 * H * D), generator=g, device=dev).to(torch.bfloat16)
    q = qkv[..., :H * D].view(1, S, H, D).transpose(1, 2)
    k = qkv[..., H * D:2 * H * D].view(1, S, H, D).transpose(1, 2)
    inv = 1.0 / (1e4 ** (torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D))
    f = torch.arange(S, device=dev, dtype=torch.float32)[:, None] * inv[None]
    emb = torch.cat([f, f], -1)[None]
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        for _ in range(2):
            fn()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * reps)]
        torch.cuda.synchronize()
        for i in range(reps):
            ev[2 * i].record(stream)
            fn()
            ev[2 * i + 1].record(stream)
        torch.cuda.synchronize()
        return sum(ev[2 * i].elapsed_time(ev[2 * i + 1]) for i in range(reps)) / reps

    ms = timed(lambda: apply_rotary_pos_emb(q, k, cos, sin, inplace=True))
    ms_hf = timed(lambda: hf_rope(q, k, cos, sin))
    nbytes = 2 * (2 * S * H * D * 2) + 2 * S * D * 2
    gbps = nbytes / (ms * 1e-3) / 1e9
    del qkv
    torch.cuda.empty_cache()
    return {"s": S, "heads": H, "ms_per_layer": round(ms, 4), "bytes": nbytes,
            "hbm_gbps": round(gbps, 1), "frac_hbm_peak": round(gbps / PEAK_HBM_GBPS, 4),
            "hf_eager_ms": round(ms_hf, 4), "speedup_vs_hf_eager": round(ms_hf / ms, 2),
            "kernel": "msa::rope_kernel<Bf16>"}


def dense_baselines(q, k, v, S, H, D, ms_sparse):
    """Same-GPU dense causal attention on the same tensors: PyTorch SDPA
    (flash / memory-efficient backends only) and this build's dense kind."""
    import torch
    import torch.nn.functional as F

    from minference import _abi

    flop = H * (S * (S + 1) // 2) * 4 * D
    res = {"flop": flop}

    def timeit(fn, reps=3):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / reps

    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel

        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            ms = timeit(lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True))
        res["sdpa_ms"] = round(ms, 3)
        res["sdpa_tflops"] = round(flop / (ms * 1e-3) / 1e12, 2)
        res["speedup_vs_sdpa"] = round(ms / ms_sparse, 2)
    except Exception as e:  # noqa: BLE001
        res["sdpa_error"] = f"{type(e).__name__}: {e}"[:200]
    torch.cuda.empty_cache()

    out = torch.empty_like(q)
    ws = _abi.workspace(_abi.attention_workspace_bytes(1, H, S, D), q.device)
    heads = [(_abi.MSA_KIND_DENSE, 0, 0, -1, 1.0 / math.sqrt(D))] * H
    ms = timeit(lambda: _abi.layer_attention(q, k, v, out, heads, ws=ws))
    res["own_dense_ms"] = round(ms, 3)
    res["own_dense_tflops"] = round(flop / (ms * 1e-3) / 1e12, 2)
    res["speedup_vs_own_dense"] = round(ms / ms_sparse, 2)
    return res


if __name__ == "__main__":
    main()
