"""Parity at the BASELINE configurations' full sizes.

config 1: stream_llm, 32 heads, S=4096, 64 sinks + 1024 band, RoPE (theta
10000) applied to Q and K first (the reference runs it on the CPU in fp32;
here the fused RoPE and the stream kernel run on bf16 inputs).
config 2: block_sparse, 32 heads, S=16384, top-100, K rows 0-3 x8.
config 3: stream_llm, 32 heads, S=65536, 128 sinks + 4096 band.
Block ids are compared with the oracle in full; outputs against the
oracle's fp64 rows on every row of every head (config 1 and config 2) or 8
rows in every query block of every head (config 3, config 2 with forced
blocks), plus every kind of tile boundary, and through size-independent
properties."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O
import row_sampling as RS
from msa_data import rope

pytestmark = pytest.mark.gpu

TOL = 2e-3


def device_qkv(dev, H, S, D=96, seed=0, sink=8.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for name in "qkv":
        x = torch.randn(1, H, S, D, generator=g, device=dev)
        if name != "v":
            for s0 in range(0, S, 8192):
                x[:, :, s0:s0 + 8192] = rope(x[:, :, s0:s0 + 8192], offset=s0)
        if name == "k" and sink:
            x[:, :, :4] *= sink
        out.append(x.to(torch.bfloat16))
    return out


def rows_for(S, extra=()):
    base = {0, 1, 63, 64, 65, 127, 128, 4095, 4096, 4097, 4224, S // 2, S - 65, S - 64, S - 1}
    return sorted(r for r in base.union(extra) if 0 <= r < S)


def oracle_rows(q, k, v, rows, visible_fn, scale):
    """Oracle output of the given rows of one head (visible_fn(row) -> key ids)."""
    out = []
    for r in rows:
        js = visible_fn(r)
        qi = q[r].astype(np.float64)
        kj = k[js].astype(np.float64)
        lg = kj @ qi * scale
        p = np.exp(lg - lg.max())
        out.append((p / p.sum()) @ v[js].astype(np.float64))
    return np.stack(out)


def check_block_heads(tag, qn, kn, vn, og, ridx, rcnt, heads, per_block):
    """per_block rows of every query block of every listed head (plus the
    boundary rows) against the oracle's fp64 rows under the head's oracle
    block ids."""
    S, D = qn.shape[2], qn.shape[3]
    scale = O.sparse_scale(D)
    extra = rows_for(S, extra=(64 * 99, 64 * 100 + 5, 64 * 200 + 17))

    def check(h):
        rows = RS.block_rows(S, h, per_block=per_block, extra=extra)
        ref = RS.head_rows_reference(qn[0, h], kn[0, h], vn[0, h], rows, RS.BLOCK, 0, 0, scale,
                                     ridx[0, h], rcnt[0, h])
        return h, rows.size, float(np.abs(og[0, h, rows] - ref).max())

    res = RS.map_heads(check, heads, tag=tag)
    print(f"{tag} {sum(r[1] for r in res)} rows, worst error {max(r[2] for r in res):.3e}",
          flush=True)
    for h, n, err in res:
        assert err < TOL, (h, n, err)


def test_cfg2_block_ids_bit_exact_and_rows(gpu_device):
    from minference.ops.block_sparse_kernel import (block_sparse_attention_with_indices,
                                                    select_block_sparse_topk_indices)

    H, S, D, topk = 32, 16384, 96, 100
    q, k, v = device_qkv(gpu_device, H, S, D, seed=2)
    print(f"[cfg2] estimator H={H} S={S} topk={topk}", flush=True)
    idx, cnt = select_block_sparse_topk_indices(q, k, topk, return_counts=True)
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    ridx, rcnt = O.select_block_sparse_topk_indices(qn, kn, topk, "bf16")
    gi = idx.cpu().numpy()
    assert np.array_equal(cnt.cpu().numpy(), rcnt)
    assert np.array_equal(rcnt, O.attend_count(ridx, S, S))
    assert np.array_equal(gi, ridx), f"{(gi != ridx).sum()} block ids differ"

    print("[cfg2] attention", flush=True)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    block_sparse_attention_with_indices(q, k, v, idx, out=out)
    og = out.cpu().numpy()
    check_block_heads("[cfg2]", qn, kn, vn, og, ridx, rcnt, range(H), per_block=64)  # every row


def test_cfg2_as_worded_forced_first_and_diagonal(gpu_device):
    """BASELINE config 2 as its text states it: top-100 of the 64-blocks with
    the diagonal and the first block always included (the selector option
    FORCE_FIRST | FORCE_DIAG, inside the top-k).  All 32 heads x 256 query
    blocks bit-exact with the oracle; then block_sparse_attention with the
    option against the oracle on 8 rows per query block of every head."""
    from minference import block_sparse_attention
    from minference.ops.block_sparse_kernel import select_block_sparse_topk_indices

    H, S, D, topk = 32, 16384, 96, 100
    q, k, v = device_qkv(gpu_device, H, S, D, seed=2)
    print(f"[cfg2 forced] estimator H={H} S={S} topk={topk}", flush=True)
    idx, cnt = select_block_sparse_topk_indices(q, k, topk, return_counts=True,
                                                force_first=True, force_diag=True)
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    ridx, rcnt = O.select_block_sparse_topk_indices(qn, kn, topk, "bf16", force_first=True,
                                                    force_diag=True)
    gi = idx.cpu().numpy()
    assert np.array_equal(cnt.cpu().numpy(), rcnt)
    assert np.array_equal(gi, ridx), f"{(gi != ridx).sum()} block ids differ"
    for bq in range(S // 64):
        row = gi[:, :, bq, :rcnt[0, 0, bq]]
        assert (row == 0).any(-1).all() and (row == bq).any(-1).all()
    # the option changes selections where the plain top-k left block 0 or bq out
    plain, _ = O.select_block_sparse_topk_indices(qn, kn, topk, "bf16")
    print(f"[cfg2 forced] rows changed by the option: "
          f"{int((plain != ridx).any(-1).sum())} of {H * (S // 64)}", flush=True)

    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    block_sparse_attention(q, k, v, topk, out=out, force_first=True, force_diag=True)
    og = out.cpu().numpy()
    check_block_heads("[cfg2 forced]", qn, kn, vn, og, ridx, rcnt, range(H), per_block=8)


def test_cfg1_rope_then_stream_all_rows(gpu_device):
    from minference import streaming_forward
    from minference.ops.rope import apply_rotary_pos_emb
    from test_rope import rope_tables

    H, S, D, n_init, n_local = 32, 4096, 96, 64, 1024
    print(f"[cfg1] RoPE + stream H={H} S={S} ({n_init}, {n_local})", flush=True)
    g = torch.Generator(device=gpu_device).manual_seed(1)
    q, k, v = (torch.randn(1, H, S, D, generator=g, device=gpu_device).to(torch.bfloat16)
               for _ in range(3))
    cos, sin = (t.to(gpu_device) for t in rope_tables(1, S, D, torch.bfloat16, theta=10000.0))
    qr, kr = apply_rotary_pos_emb(q, k, cos, sin)
    cn, sn = cos.float().cpu().numpy(), sin.float().cpu().numpy()
    qn = O.rope_rotate_half(q.float().cpu().numpy(), cn, sn, "bf16")
    kn = O.rope_rotate_half(k.float().cpu().numpy(), cn, sn, "bf16")
    assert np.array_equal(qr.float().cpu().numpy(), qn)
    assert np.array_equal(kr.float().cpu().numpy(), kn)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    streaming_forward(qr, kr, v, n_init, n_local, out=out)
    og, vn = out[0].cpu().numpy(), v[0].float().cpu().numpy()
    rows = np.arange(S)

    def check(h):   # every row of every head
        ref = RS.head_rows_reference(qn[0, h], kn[0, h], vn[h], rows, RS.STREAM, n_init,
                                     n_local, O.sparse_scale(D))
        return float(np.abs(og[h] - ref).max())

    err = max(RS.map_heads(check, range(H), tag="[cfg1]"))
    assert err < TOL, err
    vc = torch.full_like(v, -1.25)
    assert torch.all(streaming_forward(qr, kr, vc, n_init, n_local) == -1.25)


def test_cfg3_stream_rows_and_properties(gpu_device):
    from minference import dense_attention, streaming_forward

    H, S, D, n_init, n_local = 32, 65536, 96, 128, 4096
    q, k, v = device_qkv(gpu_device, H, S, D, seed=3)
    print(f"[cfg3] stream H={H} S={S} ({n_init}, {n_local})", flush=True)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    streaming_forward(q, k, v, n_init, n_local, out=out)
    scale = O.sparse_scale(D)
    extra = rows_for(S, extra=(n_local - 1, n_local, n_local + 63, n_local + 64, n_local + 127))
    qn, kn, vn, og = (t[0].float().cpu().numpy() for t in (q, k, v, out))
    del out

    def check(h):
        rows = RS.block_rows(S, h, per_block=8, extra=extra)
        ref = RS.head_rows_reference(qn[h], kn[h], vn[h], rows, RS.STREAM, n_init, n_local,
                                     scale)
        return h, rows.size, float(np.abs(og[h, rows] - ref).max())

    res = RS.map_heads(check, range(H), tag="[cfg3]")
    print(f"[cfg3] {sum(r[1] for r in res)} rows, worst error {max(r[2] for r in res):.3e}",
          flush=True)
    for h, n, err in res:
        assert err < TOL, (h, n, err)
    del qn, kn, vn, og

    # constant V: every row's output is that constant (normalisation, all rows)
    print("[cfg3] constant-V property", flush=True)
    vc = torch.full_like(v, 0.75)
    o1 = streaming_forward(q, k, vc, n_init, n_local)
    assert torch.all(o1 == 0.75)
    del o1, vc


@pytest.mark.parametrize("S", [8192, 20000])
def test_kinds_agree_where_they_coincide(gpu_device, S):
    """A stream window wider than S and a top-k of every block both reduce to
    causal dense attention; the kernels walk the same tiles in the same order,
    so the outputs agree bit for bit."""
    from minference import block_sparse_attention, dense_attention, streaming_forward

    H, D = 8, 96
    q, k, v = device_qkv(gpu_device, H, S, D, seed=4)
    scale = 128 ** -0.5
    print(f"[kinds] S={S}", flush=True)
    dense = dense_attention(q, k, v, scale=scale)
    stream = streaming_forward(q, k, v, 0, S + 1)
    block = block_sparse_attention(q, k, v, math.ceil(S / 64))
    assert torch.equal(stream, dense)
    assert torch.equal(block, dense)


@pytest.mark.parametrize("S,vsz,ssz", [(65536, 1000, 6096), (131072, 3500, 100)],
                         ids=["64k-1000-6096", "128k-3500-100"])
def test_vs_full_length_estimator_and_rows(gpu_device, S, vsz, ssz):
    """vertical_and_slash at the bench length and at MSA_VS_MAX_SEQ: estimator
    indices bit-exact with the oracle, sampled rows of the attention against
    the oracle's per-row visibility, and constant V reproduced on every row."""
    from minference.ops.vertical_slash_kernel import (vertical_and_slash_estimate,
                                                      vertical_slash_sparse_attention)

    H, D = 2, 96
    q, k, v = device_qkv(gpu_device, H, S, D, seed=S % 997)
    print(f"[vs-full] estimator S={S} ({vsz}, {ssz})", flush=True)
    vi, si = vertical_and_slash_estimate(q, k, vsz, ssz)
    qn, kn, vn = (t.float().cpu().numpy() for t in (q, k, v))
    rv, rs = O.vs_estimate(qn, kn, vsz, ssz, "bf16")
    gv, gs = vi.cpu().numpy(), si.cpu().numpy()
    assert np.array_equal(gv, rv), f"{(gv != rv).sum()} vertical ids differ"
    assert np.array_equal(gs, rs), f"{(gs != rs).sum()} slash ids differ"

    print(f"[vs-full] attention S={S}", flush=True)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    vertical_slash_sparse_attention(q, k, v, vi, si, out=out)
    rows = rows_for(S, extra=(S - 64 * 50 - 3, S - 200, S - 6096, S - 6097))
    scale = O.sparse_scale(D)
    for h in range(H):
        ref = oracle_rows(qn[0, h], kn[0, h], vn[0, h], rows,
                          lambda r, h=h: O.vs_row_visible(rv[0, h], rs[0, h], r, S), scale)
        err = np.abs(out[0, h, rows].cpu().numpy() - ref).max()
        assert err < TOL, (h, err)
    del out

    print(f"[vs-full] constant-V property S={S}", flush=True)
    vc = torch.full_like(v, -1.25)
    o1 = vertical_slash_sparse_attention(q, k, vc, vi, si)
    assert torch.all(o1 == -1.25)
