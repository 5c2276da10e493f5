"""Pins the CPU oracle (oracle/msa_oracle.py) against things other than its
own formulas: torch library routines the reference calls, brute-force loops,
closed forms and the reference tests' invariants.  CPU only."""

from __future__ import annotations

import math
import struct

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from msa_data import dtype_tag, make_qkv, np32


# ---------------------------------------------------------------------------
# scale quirk
# ---------------------------------------------------------------------------
def test_scale_quirk_phi3():
    # D=96 is padded to 128 before 1/sqrt(D) in the sparse ops; dense keeps 96
    assert O.next_allowed_head_dim(96) == 128
    assert O.sparse_scale(96) == 128 ** -0.5
    assert O.dense_scale(96) == 1 / math.sqrt(96)
    assert O.sparse_scale(64) == 64 ** -0.5
    assert O.next_allowed_head_dim(48) == 64 and O.next_allowed_head_dim(80) == 128


# ---------------------------------------------------------------------------
# rounding helpers against torch's casts
# ---------------------------------------------------------------------------
def test_bf16_round_matches_torch():
    x = torch.randn(100000, dtype=torch.float32) * torch.logspace(-30, 30, 100000)
    ref = x.to(torch.bfloat16).float().numpy()
    assert np.array_equal(O.bf16_round(x.numpy()).view(np.uint32), ref.view(np.uint32))


def test_f16_round_matches_torch():
    x = torch.randn(100000) * 100
    assert np.array_equal(O.f16_round(x.numpy()), x.half().float().numpy())


# ---------------------------------------------------------------------------
# pooling == torch's bf16/fp16 mean (the reference's library call, :240-252)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("S", [256, 300, 4096 + 17])
def test_pool_matches_torch_mean(dtype, S):
    q, _, _ = make_qkv(B=2, H=3, S_q=S, D=96, dtype=dtype, seed=S)
    pad = (-S) % 64
    qp = F.pad(q, (0, 0, 0, pad)) if pad else q
    ref = qp.reshape(2, 3, -1, 64, 96).mean(dim=3).to(torch.float32).numpy()
    got = O.pool_blocks(np32(q), dtype_tag(dtype))
    assert got.shape == ref.shape
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block,S", [(128, 300), (192, 700), (256, 1000), (320, 1500), (512, 1100)])
def test_pool_matches_torch_mean_large_blocks(dtype, block, S):
    q, _, _ = make_qkv(B=1, H=2, S_q=S, D=96, dtype=dtype, seed=S + block)
    pad = (-S) % block
    qp = F.pad(q, (0, 0, 0, pad)) if pad else q
    ref = qp.reshape(1, 2, -1, block, 96).mean(dim=3).to(torch.float32).numpy()
    got = O.pool_blocks(np32(q), dtype_tag(dtype), block)
    assert got.shape == ref.shape
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------------------------------
# selector: brute force, known answers, invariants, torch.topk
# ---------------------------------------------------------------------------
def _bf16_py(x: float) -> float:
    u = struct.unpack("<I", struct.pack("<f", x))[0]
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return struct.unpack("<f", struct.pack("<I", u))[0]


def _f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def _brute_selector(q, k, topk, scale):
    """Pure-Python selector for one head: exact sums (math.fsum), explicit
    block-causal candidate list and an explicit (-score, id) sort."""
    S, D = q.shape
    nb = -(-S // 64)

    def pool(x):
        out = []
        for b in range(nb):
            row = []
            for d in range(D):
                vals = [float(x[r, d]) if r < S else 0.0 for r in range(64 * b, 64 * b + 64)]
                row.append(_bf16_py(_f32(_f32(math.fsum(vals)) / 64.0)))
            out.append(row)
        return out

    qp, kp = pool(q), pool(k)
    ids, cnts = [], []
    for bq in range(nb):
        cands = []
        for bk in range(bq + 1):
            s = _f32(_f32(math.fsum(a * b for a, b in zip(qp[bq], kp[bk]))) * _f32(scale))
            cands.append((-s, bk))
        cands.sort()
        c = min(topk, bq + 1)
        sel = sorted(bk for _, bk in cands[:c])
        sel += [bq + 1 + i for i in range(min(topk, nb) - c)]
        ids.append(sel)
        cnts.append(c)
    return np.array(ids), np.array(cnts)


@pytest.mark.parametrize("S,topk", [(640, 3), (600, 1), (512, 8), (448, 100)])
def test_selector_bruteforce(S, topk):
    q, k, _ = make_qkv(B=1, H=2, S_q=S, D=32, dtype=torch.bfloat16, seed=7 + S)
    scale = O.sparse_scale(32)
    idx, cnt = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, "bf16", scale)
    for h in range(2):
        bi, bc = _brute_selector(np32(q)[0, h], np32(k)[0, h], topk, scale)
        assert np.array_equal(idx[0, h], bi)
        assert np.array_equal(cnt[0, h], bc)


def test_selector_known_answer_monotone():
    # pooled K block b = (b+1) * e0, pooled Q = e0 -> score grows with b:
    # the top-k of row bq are its last k causal blocks
    S, D = 64 * 12, 64
    k = torch.zeros(1, 1, S, D)
    for b in range(12):
        k[0, 0, 64 * b:64 * b + 64, 0] = float(b + 1)
    q = torch.zeros(1, 1, S, D)
    q[..., 0] = 1.0
    idx, cnt = O.select_block_sparse_topk_indices(q.numpy(), k.numpy(), 4, "bf16")
    for bq in range(12):
        c = min(4, bq + 1)
        assert cnt[0, 0, bq] == c
        assert list(idx[0, 0, bq, :c]) == list(range(bq + 1 - c, bq + 1))


def test_selector_known_answer_ties_to_lower_id():
    # identical K blocks -> all causal scores tie -> the lowest ids win
    S, D = 64 * 10, 64
    blk = torch.randn(64, D)
    k = blk.repeat(10, 1)[None, None]
    q = torch.randn(1, 1, S, D)
    idx, cnt = O.select_block_sparse_topk_indices(q.numpy(), k.numpy(), 3, "bf16")
    for bq in range(10):
        c = min(3, bq + 1)
        assert list(idx[0, 0, bq, :c]) == list(range(c))
        assert list(idx[0, 0, bq, c:]) == list(range(bq + 1, bq + 1 + 3 - c))


def test_selector_forced_known_answer():
    """Decreasing pooled scores (K block b = (12 - b) * e0, Q = e0): the plain
    top-k of row bq is its first k causal blocks; with the diagonal forced the
    row keeps bq and the first k-1; with block 0 forced nothing changes (it is
    already first); top-1 with both flags keeps block 0 (lower id)."""
    S, D = 64 * 12, 64
    k = torch.zeros(1, 1, S, D)
    for b in range(12):
        k[0, 0, 64 * b:64 * b + 64, 0] = float(12 - b)
    q = torch.zeros(1, 1, S, D)
    q[..., 0] = 1.0
    qn, kn = q.numpy(), k.numpy()
    plain, _ = O.select_block_sparse_topk_indices(qn, kn, 4, "bf16")
    diag, cd = O.select_block_sparse_topk_indices(qn, kn, 4, "bf16", force_diag=True)
    first, _ = O.select_block_sparse_topk_indices(qn, kn, 4, "bf16", force_first=True)
    both1, _ = O.select_block_sparse_topk_indices(qn, kn, 1, "bf16", force_first=True,
                                                  force_diag=True)
    for bq in range(12):
        c = min(4, bq + 1)
        assert list(plain[0, 0, bq, :c]) == list(range(c))
        assert list(first[0, 0, bq, :c]) == list(range(c))
        want = list(range(c)) if bq < 4 else [0, 1, 2, bq]
        assert list(diag[0, 0, bq, :c]) == want and cd[0, 0, bq] == c
        assert list(both1[0, 0, bq, :1]) == [0]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_selector_nan_order_vs_torch_topk(seed):
    """NaN scores rank above every number, +inf included, with ties between
    NaNs to the lower id: the selection equals torch.topk's (the library
    call of the reference, block_sparse_kernel_npu.py:262) on rows of
    distinct finite values, +-inf and NaN entries."""
    rng = np.random.default_rng(seed)
    n_bq = n_bk = 40
    sc = rng.permutation(n_bq * n_bk).reshape(n_bq, n_bk).astype(np.float32) * 1e-3 - 0.8
    sc[rng.random(sc.shape) < 0.08] = np.nan
    sc[rng.random(sc.shape) < 0.03] = np.inf
    sc[rng.random(sc.shape) < 0.03] = -np.inf
    for topk in (1, 3, 7):
        idx, cnt = O.select_topk(sc[None], topk)
        for bq in range(n_bq):
            n = bq + 1
            row = torch.from_numpy(sc[bq, :n].copy())
            # torch.topk orders equal values (+-inf here) by its own rule:
            # compare on rows where the k-th pick is not tied
            vals, ids = torch.topk(row, min(topk, n))
            kth = vals[-1].item()
            rest = row[[i for i in range(n) if i not in ids.tolist()]]
            if (not math.isnan(kth) and (rest == kth).any()) or (
                    math.isnan(kth) and torch.isnan(rest).any()):
                continue
            assert sorted(ids.tolist()) == list(idx[0, bq, :cnt[0, bq]]), (topk, bq)


def test_selector_forced_above_nan():
    """Forced ids rank above NaN scores (this build's selector option)."""
    sc = np.full((1, 6, 6), np.nan, dtype=np.float32)
    idx, cnt = O.select_topk(sc, 2, force_first=True, force_diag=True)
    for bq in range(6):
        want = [0] if bq == 0 else [0, bq]
        assert list(idx[0, bq, :cnt[0, bq]]) == want


@pytest.mark.parametrize("first,diag,topk", [(True, True, 5), (False, True, 3), (True, False, 1),
                                             (True, True, 2)])
def test_selector_forced_bruteforce(first, diag, topk):
    """Forced selection = the forced ids plus the brute-force top-(k - |forced|)
    of the other causal blocks (ties -> lower id), written without the +inf
    device the oracle uses."""
    S = 64 * 9 + 17
    q, k, _ = make_qkv(B=1, H=2, S_q=S, D=32, dtype=torch.bfloat16, seed=41)
    scale = O.sparse_scale(32)
    idx, cnt = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, "bf16", scale,
                                                  force_first=first, force_diag=diag)
    nb = -(-S // 64)
    for h in range(2):
        qp = O.pool_blocks(np32(q)[0, h], "bf16").astype(np.float64)
        kp = O.pool_blocks(np32(k)[0, h], "bf16").astype(np.float64)
        for bq in range(nb):
            forced = []
            if first:
                forced.append(0)
            if diag and bq not in forced:
                forced.append(bq)
            kk = min(topk, bq + 1)
            forced = sorted(forced)[:kk]
            rest = [b for b in range(bq + 1) if b not in forced]
            sc = {b: float(np.float32(np.float32(math.fsum(qp[bq] * kp[b])) * np.float32(scale)))
                  for b in rest}
            rest.sort(key=lambda b: (-sc[b], b))
            want = sorted(forced + rest[:kk - len(forced)])
            assert cnt[0, h, bq] == kk
            assert list(idx[0, h, bq, :kk]) == want, (h, bq)


@pytest.mark.parametrize("topk,S", [(1, 256), (2, 256), (4, 512), (100, 256)])
def test_selector_invariants(topk, S):
    """Reference tests/test_block_sparse_kernel.py:186-211: sorted, clamped,
    visible count == min(topk, bq+1)."""
    q, k, _ = make_qkv(B=1, H=2, S_q=S, D=64, dtype=torch.float32, seed=23)
    idx, cnt = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, "fp32")
    n = S // 64
    kk = min(topk, n)
    assert idx.shape == (1, 2, n, kk)
    assert (idx[..., 1:] >= idx[..., :-1]).all()
    vis = (idx <= np.arange(n)[None, None, :, None]).sum(-1)
    assert np.array_equal(vis, np.minimum(kk, np.arange(n) + 1)[None, None].repeat(2, 1))
    assert np.array_equal(cnt, vis)


@pytest.mark.parametrize("S,topk", [(4096, 16), (2048 + 64 * 3, 7)])
def test_selector_vs_torch_topk(S, topk):
    """The reference's selector steps as torch library calls (bf16 mean,
    fp32 matmul, -inf mask, topk, sort; :240-263): the causal sets agree with
    the oracle except where the k-th / (k+1)-th scores are a near tie."""
    q, k, _ = make_qkv(B=1, H=4, S_q=S, D=96, dtype=torch.bfloat16, seed=5, sink_scale=8.0)
    D = 96
    scale = 128 ** -0.5
    qp = q.reshape(1, 4, -1, 64, D).mean(dim=3).float()
    kp = k.reshape(1, 4, -1, 64, D).mean(dim=3).float()
    sc = torch.matmul(qp, kp.transpose(-1, -2)) * scale
    nb = sc.shape[-1]
    causal = torch.arange(nb)[:, None] >= torch.arange(nb)[None, :]
    sc = sc.masked_fill(~causal, float("-inf"))
    ref = torch.topk(sc, min(topk, nb), dim=-1).indices.sort(dim=-1).values.numpy()
    idx, cnt = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, "bf16", scale)
    osc = O.block_scores(O.pool_blocks(np32(q), "bf16"), O.pool_blocks(np32(k), "bf16"), scale)
    mismatches = 0
    for h in range(4):
        for bq in range(nb):
            c = cnt[0, h, bq]
            a = set(idx[0, h, bq, :c].tolist())
            b = set(x for x in ref[0, h, bq].tolist() if x <= bq)
            if a != b:
                mismatches += 1
                row = np.sort(osc[0, h, bq, :bq + 1].astype(np.float64))[::-1]
                gap = abs(row[c - 1] - row[c])
                assert gap <= 1e-6 * max(1.0, abs(row[c - 1])), (h, bq, a ^ b, gap)
    assert mismatches <= 2


# ---------------------------------------------------------------------------
# streaming
# ---------------------------------------------------------------------------
def _brute_stream_row(q, k, v, i, s_q, s_k, n_init, n_local, scale):
    a = s_k - s_q + i
    vis = [j for j in range(s_k) if j <= a and (j > a - n_local or j < n_init)]
    if not vis:
        return np.zeros(q.shape[-1])
    lg = np.array([float(np.dot(q[i].astype(np.float64), k[j].astype(np.float64))) * scale
                   for j in vis])
    p = np.exp(lg - lg.max())
    p /= p.sum()
    return (p[:, None] * v[vis].astype(np.float64)).sum(0)


# (n_init, n_local, s_q, s_k) from reference tests/test_streaming_kernel.py:127-147
STREAM_CASES = [
    (64, 512, 256, 256),
    (64, 512, 128, 128),
    (4, 8, 9, 9),
    (0, 16, 32, 64),
    (128, 512, 512, 1024),
    (128, 256, 256, 512),
    (400, 128, 128, 512),
    (64, 1, 128, 256),
    (1, 64, 128, 256),
]


@pytest.mark.parametrize("case", STREAM_CASES)
def test_streaming_vs_bruteforce(case):
    n_init, n_local, s_q, s_k = case
    q, k, v = make_qkv(B=1, H=1, S_q=s_q, S_k=s_k, D=64, dtype=torch.float32, seed=42)
    qn, kn, vn = np32(q)[0, 0], np32(k)[0, 0], np32(v)[0, 0]
    out = O.streaming_attention(np32(q), np32(k), np32(v), n_init, n_local)[0, 0]
    scale = O.sparse_scale(64)
    rows = sorted(set([0, 1, s_q // 2, s_q - 1] + list(range(0, s_q, max(1, s_q // 16)))))
    for i in rows:
        ref = _brute_stream_row(qn, kn, vn, i, s_q, s_k, n_init, n_local, scale)
        assert np.abs(out[i] - ref).max() < 1e-9


def _uniform_mean(v, visible):
    """Closed form for Q = 0: softmax is uniform over the visible set."""
    cnt = visible.sum(-1, keepdims=True)
    return np.where(cnt > 0, (visible.astype(np.float64) @ v.astype(np.float64)) / np.maximum(cnt, 1), 0.0)


@pytest.mark.parametrize("case", STREAM_CASES)
def test_streaming_q0_closed_form(case):
    n_init, n_local, s_q, s_k = case
    _, k, v = make_qkv(B=1, H=1, S_q=s_q, S_k=s_k, D=64, dtype=torch.float32, seed=3)
    q = np.zeros((1, 1, s_q, 64), np.float32)
    out = O.streaming_attention(q, np32(k), np32(v), n_init, n_local)[0, 0]
    # visible set built independently: cumulative windows by explicit loops
    vis = np.zeros((s_q, s_k), bool)
    for i in range(s_q):
        a = s_k - s_q + i
        lo = max(0, a - n_local + 1)
        vis[i, lo:a + 1] = True
        vis[i, :min(n_init, a + 1)] = True
    assert np.abs(out - _uniform_mean(np32(v)[0, 0], vis)).max() < 1e-12


def test_streaming_wide_band_equals_causal_dense():
    q, k, v = make_qkv(B=1, H=2, S_q=192, D=64, dtype=torch.float32, seed=9)
    s = O.sparse_scale(64)
    a = O.streaming_attention(np32(q), np32(k), np32(v), 0, 10**6, scale=s)
    b = O.dense_causal(np32(q), np32(k), np32(v), scale=s)
    assert np.abs(a - b).max() < 1e-12


def test_streaming_lse_merge_identity():
    """Sink part and band part as separate softmaxes merged by log-sum-exp
    (the reference's NPU path, streaming_kernel_npu.py:322-341) equal the
    single masked softmax."""
    n_init, n_local, S = 96, 128, 512
    q, k, v = make_qkv(B=1, H=1, S_q=S, D=64, dtype=torch.float32, seed=11)
    qn, kn, vn = (np32(t)[0, 0].astype(np.float64) for t in (q, k, v))
    sc = O.sparse_scale(64)
    lg = qn @ kn.T * sc
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    band = (j <= i) & (j > i - n_local)
    sink = (j < n_init) & (j < i - n_local + 1)

    def part(mask):
        x = np.where(mask, lg, -np.inf)
        m = x.max(-1, keepdims=True)
        m = np.where(np.isfinite(m), m, -1e300)
        p = np.exp(x - m)
        l = p.sum(-1, keepdims=True)
        o = (p @ vn) / np.where(l > 0, l, 1)
        return m, l, o

    m1, l1, o1 = part(band)
    m2, l2, o2 = part(sink)
    m = np.maximum(m1, m2)
    a1, a2 = np.exp(m1 - m) * l1, np.exp(m2 - m) * l2
    merged = (a1 * o1 + a2 * o2) / (a1 + a2)
    out = O.streaming_attention(np32(q), np32(k), np32(v), n_init, n_local)[0, 0]
    assert np.abs(out - merged).max() < 1e-12


# ---------------------------------------------------------------------------
# block sparse given indices, dense
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("S", [128, 256, 300])
def test_block_full_topk_equals_dense(S):
    """Reference tests/test_block_sparse_kernel.py:237-256."""
    q, k, v = make_qkv(B=1, H=2, S_q=S, D=64, dtype=torch.float32, seed=0)
    nb = -(-S // 64)
    idx, _ = O.select_block_sparse_topk_indices(np32(q), np32(k), nb, "fp32")
    s = O.sparse_scale(64)
    a = O.block_sparse_from_indices(np32(q), np32(k), np32(v), idx, scale=s)
    b = O.dense_causal(np32(q), np32(k), np32(v), scale=s)
    assert np.abs(a - b).max() < 1e-12


@pytest.mark.parametrize("s_q,s_k", [(128, 512), (100, 700), (300, 2000)])
def test_block_chunked_full_topk_equals_dense(s_q, s_k):
    """Chunked prefill (S_q < S_k): with top-k = n_kb every id row holds all
    blocks (the causal picks plus the q-frame -inf picks), so the token mask
    reduces to the absolute causal mask and the output to causal dense."""
    q, k, v = make_qkv(B=1, H=2, S_q=s_q, S_k=s_k, D=64, dtype=torch.float32, seed=s_q)
    nb = -(-s_k // 64)
    idx, cnt = O.select_block_sparse_topk_indices(np32(q), np32(k), nb, "fp32")
    assert (np.sort(idx, -1) == np.arange(nb)).all()
    s = O.sparse_scale(64)
    a = O.block_sparse_from_indices(np32(q), np32(k), np32(v), idx, scale=s)
    b = O.dense_causal(np32(q), np32(k), np32(v), scale=s)
    assert np.abs(a - b).max() < 1e-12


@pytest.mark.parametrize("s_q,s_k,topk", [(64, 64, 1), (256, 256, 3), (100, 700, 3), (128, 512, 5),
                                          (70, 1000, 16), (300, 2000, 40)])
def test_attend_count_bruteforce(s_q, s_k, topk):
    """attend_count against the token mask itself: id b of block row bq counts
    iff some (row of bq, key of b) pair is visible."""
    q, k, _ = make_qkv(B=1, H=1, S_q=s_q, S_k=s_k, D=32, dtype=torch.float32, seed=topk)
    idx, cnt = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, "fp32")
    got = O.attend_count(idx, s_q, s_k)[0, 0]
    for bq in range(idx.shape[2]):
        vis = O.block_token_visible(idx[0, 0], s_q, s_k)[64 * bq:64 * bq + 64]
        seen = [b for b in idx[0, 0, bq] if vis[:, 64 * b:64 * b + 64].any()]
        assert got[bq] == len(seen)
        assert list(idx[0, 0, bq, :got[bq]]) == seen  # a prefix of the row
        if s_q == s_k:
            assert got[bq] == cnt[0, 0, bq] == min(topk, bq + 1)


def test_block_q0_closed_form_and_bruteforce():
    S, topk = 448, 3
    q, k, v = make_qkv(B=1, H=1, S_q=S, D=64, dtype=torch.bfloat16, seed=4)
    idx, _ = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, "bf16")
    nb = S // 64
    vis = np.zeros((S, S), bool)
    for i in range(S):
        for bk in idx[0, 0, i // 64]:
            for j in range(64 * bk, min(S, 64 * bk + 64)):
                if j <= i:
                    vis[i, j] = True
    qz = np.zeros((1, 1, S, 64), np.float32)
    out0 = O.block_sparse_from_indices(qz, np32(k), np32(v), idx)[0, 0]
    assert np.abs(out0 - _uniform_mean(np32(v)[0, 0], vis)).max() < 1e-12
    out = O.block_sparse_from_indices(np32(q), np32(k), np32(v), idx)[0, 0]
    sc = O.sparse_scale(64)
    qn, kn, vn = (np32(t)[0, 0].astype(np.float64) for t in (q, k, v))
    for i in (0, 63, 64, 200, S - 1):
        js = np.nonzero(vis[i])[0]
        lg = qn[i] @ kn[js].T * sc
        p = np.exp(lg - lg.max())
        ref = (p / p.sum()) @ vn[js]
        assert np.abs(out[i] - ref).max() < 1e-12
    assert nb == 7


@pytest.mark.parametrize("s_q,s_k", [(256, 256), (100, 300), (300, 100)])
def test_dense_noncausal_vs_torch_sdpa(s_q, s_k):
    """causal=False (attention.py:181-186, :221-230): every key for every
    query, S_q > S_k included."""
    q, k, v = make_qkv(B=1, H=2, S_q=s_q, S_k=s_k, D=64, dtype=torch.float32, seed=3,
                       use_rope=False)
    out = O.dense_causal(np32(q), np32(k), np32(v), causal=False)
    ref = F.scaled_dot_product_attention(q.double(), k.double(), v.double(), scale=64 ** -0.5)
    assert np.abs(out - ref.numpy()).max() < 1e-12


@pytest.mark.parametrize("s_q,s_k", [(256, 256), (100, 300)])
def test_dense_vs_torch_sdpa(s_q, s_k):
    q, k, v = make_qkv(B=1, H=2, S_q=s_q, S_k=s_k, D=96, dtype=torch.float32, seed=1)
    out = O.dense_causal(np32(q), np32(k), np32(v))
    mask = torch.arange(s_k)[None, :] <= (torch.arange(s_q)[:, None] + s_k - s_q)
    ref = F.scaled_dot_product_attention(q.double(), k.double(), v.double(), attn_mask=mask,
                                         scale=96 ** -0.5)
    assert np.abs(out - ref.numpy()).max() < 1e-12


# ---------------------------------------------------------------------------
# row-sampled attention (the full-length GPU checks' reference)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("group", [1, 7, 64])
def test_rows_attention_equals_full_heads(group):
    """Every row, grouped any way, equals the pinned full-head functions;
    a rule with a wrong sign or an off-by-one at the band or block edge
    would move rows at those edges."""
    S, D = 777, 64
    q, k, v = make_qkv(B=1, H=1, S_q=S, D=D, dtype=torch.bfloat16, seed=6)
    qn, kn, vn = np32(q), np32(k), np32(v)
    sc = O.sparse_scale(D)
    rows = np.arange(S)
    for n_init, n_local in [(0, 100), (64, 128), (3, 1), (100, 2000)]:
        ref = O.streaming_attention(qn, kn, vn, n_init, n_local)[0, 0]
        vis, keys = O.stream_rows_visible(n_init, n_local)
        got = O.rows_attention(qn[0, 0], kn[0, 0], vn[0, 0], rows, vis, sc, keys=keys,
                               group=group)
        assert np.abs(got - ref).max() < 1e-12, (n_init, n_local)
        got = O.rows_attention(qn[0, 0], kn[0, 0], vn[0, 0], rows, vis, sc, group=group)
        assert np.abs(got - ref).max() < 1e-12, (n_init, n_local)
    for topk in (1, 3, 13):
        idx, cnt = O.select_block_sparse_topk_indices(qn, kn, topk, "bf16")
        ref = O.block_sparse_from_indices(qn, kn, vn, idx)[0, 0]
        vis, keys = O.block_rows_visible(idx[0, 0], cnt[0, 0], S)
        for kf in (keys, None):
            got = O.rows_attention(qn[0, 0], kn[0, 0], vn[0, 0], rows, vis, sc, keys=kf,
                                   group=group)
            assert np.abs(got - ref).max() < 1e-12, topk
    ref = O.dense_causal(qn, kn, vn, scale=sc)[0, 0]
    got = O.rows_attention(qn[0, 0], kn[0, 0], vn[0, 0], rows, O.causal_rows_visible, sc,
                           group=group)
    assert np.abs(got - ref).max() < 1e-12


def test_block_rows_visible_counts_and_invalid_ids():
    """Padding past cnt and ids outside [0, n_kv_blocks) see nothing; a
    sampled row sees exactly its listed blocks' keys up to itself."""
    S = 300
    idx = np.array([[0, -1, 9], [1, 0, 2], [2, 4, 7], [3, 0, 1], [4, 1, 0]], np.int32)
    cnt = np.array([1, 2, 3, 2, 3], np.int32)
    vis, keys_of = O.block_rows_visible(idx, cnt, S)
    keys = np.arange(S)
    for r in (0, 63, 64, 130, 191, 250, 299):
        want = set()
        for b in idx[r // 64, :cnt[r // 64]]:
            if 0 <= b < 5:
                want |= {j for j in range(64 * b, min(S, 64 * b + 64)) if j <= r}
        got = set(np.nonzero(vis(np.array([r]), keys)[0])[0].tolist())
        assert got == want, r
        assert want <= set(keys_of(np.array([r])).tolist()), r


# ---------------------------------------------------------------------------
# algorithmic work counts (closed forms for the benchmark configurations)
# ---------------------------------------------------------------------------
def test_work_counts_small_bruteforce():
    for S, ni, nl in [(300, 20, 50), (1000, 128, 256), (64, 0, 64)]:
        assert O.stream_pairs(S, ni, nl) == int(O.stream_visible(S, S, ni, nl).sum())
    for S, k in [(640, 3), (1000, 100)]:
        nb = -(-S // 64)
        assert O.block_tiles(S, k) == sum(min(k, b + 1) for b in range(nb))


def test_work_counts_baseline_configs():
    assert O.stream_pairs(4096, 64, 1024) == 3_865_120
    assert O.block_tiles(16384, 100) == 20_650
    assert O.stream_pairs(65536, 128, 4096) == 267_905_088
    assert O.stream_pairs(32768, 128, 4096) == 129_493_056
    assert O.block_tiles(32768, 100) == 46_250
    assert O.stream_pairs(131072, 128, 8192) == 1_055_912_000
    assert O.block_tiles(131072, 160) == 314_960
    assert O.causal_pairs(32768) == 536_887_296
