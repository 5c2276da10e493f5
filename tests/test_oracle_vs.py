"""vertical_and_slash oracle pins (CPU).

The estimator (minference_forward.py:140-167), the token mask of the
reference's production path (vertical_slash_kernel_npu.py:282-367) and the
attention built on it are checked against brute force, closed forms, the
reference's own test properties (tests/test_vertical_slash_kernel.py) and
the reference formula evaluated with torch, none of which reuse the oracle's
code."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O
from msa_data import make_qkv, np32


# ---------------------------------------------------------------------------
# estimator
# ---------------------------------------------------------------------------
def _brute_scores(q, k, dtype):
    """Pure-Python loops: scores with math.fsum, softmax with math.exp, column
    sums and diagonal sums by walking every (row, column) pair."""
    S, D = k.shape
    n = min(64, S)
    rows = []
    for r in range(n):
        qi = [float(x) for x in q[S - n + r]]
        xs = []
        for j in range(S):
            if j - (S - n) > r:
                xs.append(-math.inf)
                continue
            d = math.fsum(qi[e] * float(k[j, e]) for e in range(D))
            a = O.round_to(np.array([d], np.float32), dtype)[0]
            xs.append(float(O.round_to(np.array([a / np.float32(math.sqrt(D))], np.float32), dtype)[0]))
        m = max(xs)
        es = [math.exp(x - m) if x != -math.inf else 0.0 for x in xs]
        tot = math.fsum(es)
        rows.append([e / tot for e in es])
    vert = [math.fsum(rows[r][j] for r in range(n)) for j in range(S)]
    diag = [[] for _ in range(S)]
    for r in range(n):
        for j in range(S):
            t = j - r + n - 1          # diagonal of (row r, column j) in the truncated output
            if 0 <= t < S:
                diag[t].append(rows[r][j])
    slash = [math.fsum(d) for d in diag]
    vert = np.array(vert, dtype=np.float32)
    slash = np.array(slash, dtype=np.float32)
    vert[:30] = np.inf
    slash[max(0, S - 100):] = np.inf
    return vert, slash


@pytest.mark.parametrize("S,D,dtype", [(8, 8, "bf16"), (70, 16, "bf16"), (130, 32, "fp16"),
                                       (200, 8, "fp32")])
def test_vs_scores_bruteforce(S, D, dtype):
    tdt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dtype]
    q, k, _ = make_qkv(B=1, H=1, S_q=S, D=D, dtype=tdt, seed=S)
    qn, kn = np32(q)[0, 0], np32(k)[0, 0]
    vert, slash = O.vs_scores(qn, kn, dtype)
    bv, bs = _brute_scores(qn, kn, dtype)
    fin = np.isfinite(bv)
    assert (np.isfinite(vert) == fin).all() and (np.isfinite(slash) == np.isfinite(bs)).all()
    if fin.any():
        assert np.abs(vert[fin] - bv[fin]).max() <= 1e-6 * np.abs(bv[fin]).max()
    fs = np.isfinite(bs)
    if fs.any():
        assert np.abs(slash[fs] - bs[fs]).max() <= 1e-6 * np.abs(bs[fs]).max()


def _torch_reference_sums(q, k, vsz, ssz):
    """The reference's estimator steps (:148-164) written with torch ops on a
    [1, 1, S, D] tensor pair; the diagonal sums via an explicit index map."""
    S, D = q.shape[-2], q.shape[-1]
    n = min(64, S)
    qk = torch.matmul(q[..., -n:, :], k.transpose(-2, -1)) / math.sqrt(D)
    r = torch.arange(n)[:, None]
    c = torch.arange(n)[None, :]
    qk[..., -n:] = torch.where(r >= c, qk[..., -n:], float("-inf"))
    p = torch.softmax(qk, dim=-1, dtype=torch.float32)[0, 0]
    vertical = p.sum(0)
    vertical[:30] = float("inf")
    t_of = torch.arange(S)[None, :] - torch.arange(n)[:, None] + n - 1   # diagonal of (r, j)
    slash = torch.zeros(S + n, dtype=torch.float32)
    slash.index_add_(0, (t_of.clamp(min=0, max=S + n - 1)).flatten(),
                     torch.where((t_of >= 0) & (t_of < S), p, torch.zeros_like(p)).flatten())
    slash = slash[:S]
    slash[max(0, S - 100):] = float("inf")
    return vertical.double().numpy(), slash.double().numpy()


def _same_selection(sel, ref_sel, vals, rel=1e-5):
    """Equal sets, except swaps at the top-k boundary between equal values
    (torch.topk's choice among exact ties, e.g. more forced +inf entries than
    k) or values closer than ``rel`` (fp32 softmax / summation noise in the
    torch evaluation)."""
    a, b = set(sel.tolist()), set(ref_sel.tolist())
    if a == b:
        return True
    only_a, only_b = a - b, b - a
    worst_in = min(vals[list(only_a)])
    best_out = max(vals[list(only_b)])
    if worst_in == best_out:
        return True
    return abs(worst_in - best_out) <= rel * abs(best_out)


@pytest.mark.parametrize("S,vsz,ssz", [(256, 60, 80), (1000, 100, 300), (2048, 500, 120),
                                       (97, 30, 50)])
def test_vs_estimate_vs_torch_formula(S, vsz, ssz):
    q, k, _ = make_qkv(B=1, H=2, S_q=S, D=96, dtype=torch.bfloat16, seed=S + vsz)
    v_idx, s_idx = O.vs_estimate(np32(q), np32(k), vsz, ssz, "bf16")
    nv, ns = O.vs_sizes(S, vsz, ssz)
    for h in range(2):
        tv, ts = _torch_reference_sums(q[:, h:h + 1], k[:, h:h + 1], vsz, ssz)
        ref_v = np.sort(torch.topk(torch.from_numpy(tv), nv).indices.numpy())
        ref_t = torch.topk(torch.from_numpy(ts), ns).indices.numpy()
        assert _same_selection(v_idx[0, h], ref_v, tv)
        assert _same_selection(S - 1 - s_idx[0, h], ref_t, ts)


def test_vs_estimate_invariants():
    S = 1500
    q, k, _ = make_qkv(B=2, H=3, S_q=S, D=64, dtype=torch.float16, seed=3, sink_scale=8.0)
    v_idx, s_idx = O.vs_estimate(np32(q), np32(k), 200, 400, "fp16")
    assert v_idx.shape == (2, 3, 200) and s_idx.shape == (2, 3, 400)
    for b in range(2):
        for h in range(3):
            v, s = v_idx[b, h], s_idx[b, h]
            assert (np.diff(v) > 0).all() and v[0] >= 0 and v[-1] < S
            assert (np.diff(s) < 0).all() and s[-1] >= 0 and s[0] < S
            assert set(range(30)) <= set(v.tolist())          # forced sink columns
            assert set(range(100)) <= set(s.tolist())         # forced local diagonals


def test_vs_estimate_zero_query_closed_form():
    """q = 0: every visible score is 0, so row r (absolute S - n + r) spreads
    1 / (S - n + r + 1) over its columns.  Column j < S - n collects
    sum_r 1 / (S - n + r + 1), the same for all such j, so the ties go to the
    lowest columns; diagonal t collects that value over its rows."""
    S, D, n = 300, 32, 64
    q = np.zeros((1, 1, S, D), np.float32)
    _, k, _ = make_qkv(B=1, H=1, S_q=S, D=D, dtype=torch.bfloat16, seed=1)
    vert, slash = O.vs_scores(q[0, 0], np32(k)[0, 0], "bf16")
    w = [1.0 / (S - n + r + 1) for r in range(n)]
    assert abs(vert[100] - math.fsum(w)) < 1e-6
    for t in (10, 63, 64, 150):
        exp_t = math.fsum(w[r] for r in range(n) if 0 <= r + t + 1 - n < S)
        assert abs(slash[t] - exp_t) < 1e-6, t
    v_idx, s_idx = O.vs_estimate(q, np32(k), 50, 120, "bf16")
    assert list(v_idx[0, 0]) == list(range(50))
    # slash: the last 100 diagonals are forced; diagonals with more rows weigh more
    t_sel = S - 1 - s_idx[0, 0]
    assert set(range(S - 100, S)) <= set(t_sel.tolist())


# ---------------------------------------------------------------------------
# token mask
# ---------------------------------------------------------------------------
def _visible_dual(v_idx, s_idx, S):
    """Same mask from the other side: key j of block bq is in a slash window
    iff some slash s lies in the window of s values that reach it."""
    vis = np.zeros((S, S), dtype=bool)
    sset = set(int(s) for s in s_idx)
    vset = set(min(max(int(c), 0), S - 1) for c in v_idx)
    for i in range(S):
        end_m = 64 * (i // 64 + 1)
        for j in range(i + 1):
            hit = j in vset
            if not hit:
                # unclamped windows [end_m - s - 64, end_m - s) hold j iff
                # end_m - 64 - j <= s <= end_m - 1 - j; windows clamped to
                # [0, 64) (end_m - s < 64) hold every j < 64
                for s in sset:
                    if s >= end_m:
                        continue
                    hi = min(max(end_m - s, 64), S)
                    if end_m - s >= 64 and hi == end_m - s:
                        hit = end_m - 64 - j <= s <= end_m - 1 - j
                    else:
                        hit = max(hi - 64, 0) <= j < hi
                    if hit:
                        break
            vis[i, j] = hit
    return vis


@pytest.mark.parametrize("S,nv,ns,seed", [(130, 35, 60, 0), (256, 40, 70, 1), (200, 30, 150, 2)])
def test_vs_token_visible_dual_form(S, nv, ns, seed):
    g = np.random.default_rng(seed)
    v = np.sort(g.choice(S, nv, replace=False))
    s = np.sort(g.choice(S, ns, replace=False))[::-1]
    assert (O.vs_token_visible(v, s, S, S) == _visible_dual(v, s, S)).all()


@pytest.mark.parametrize("S,nv,ns,seed", [(130, 35, 60, 0), (256, 40, 70, 1), (200, 30, 150, 2),
                                         (300, 20, 40, 3)])
def test_vs_row_visible_equals_mask_rows(S, nv, ns, seed):
    """The per-row form used at full sizes gives exactly the rows of the
    token mask (which the slash-side dual form pins above), including
    out-of-range and repeated indices."""
    g = np.random.default_rng(seed)
    v = np.sort(g.integers(-10, S + 10, nv))
    s = np.sort(g.integers(-20, S + 20, ns))[::-1]
    vis = O.vs_token_visible(v, s, S, S)
    for r in range(S):
        assert np.array_equal(O.vs_row_visible(v, s, r, S), np.nonzero(vis[r])[0]), r


def test_vs_token_visible_reference_properties():
    """tests/test_vertical_slash_kernel.py:207-238: the strict upper triangle is
    masked, the diagonal is not all masked, the 30 sink columns are visible to
    every row at or below them; plus: every selected slash is visible along
    its whole diagonal, and full index sets give the causal mask."""
    S = 256
    g = np.random.default_rng(7)
    v = np.sort(np.concatenate([np.arange(30), 30 + g.choice(S - 30, 20, replace=False)]))
    s = np.sort(np.concatenate([np.arange(100), 100 + g.choice(S - 100, 40, replace=False)]))[::-1]
    vis = O.vs_token_visible(v, s, S, S)
    i, j = np.arange(S)[:, None], np.arange(S)[None, :]
    assert not vis[j > i].any()
    assert vis.diagonal().any()
    for col in range(30):
        assert vis[col:, col].all()
    for sd in s:
        rows = np.arange(sd, S)
        assert vis[rows, rows - sd].all()
    full = O.vs_token_visible(np.arange(S), np.arange(S)[::-1], S, S)
    assert (full == (j <= i)).all()


def test_vs_token_visible_clamps_out_of_range_indices():
    """Vertical ids are clamped into [0, S) and slash windows into [0, S)
    (vertical_slash_kernel_npu.py:332-349)."""
    S = 128
    vis = O.vs_token_visible(np.array([-5, 500]), np.array([1000, -3]), S, S)
    # -5 -> column 0, 500 -> column 127; slash 1000 never valid; slash -3 reaches keys
    # [end_m + 3 - 64, end_m + 3) -> future keys are masked by causality
    assert vis[:, 0].all() and vis[127, 127]
    end_m = 64
    for r in range(64):
        lo, hi = end_m + 3 - 64, end_m + 3
        exp = np.zeros(S, bool)
        exp[max(lo, 0):min(hi, S)] = True
        exp[0] = True
        exp[127] = True
        exp &= np.arange(S) <= r
        assert (vis[r] == exp).all(), r


# ---------------------------------------------------------------------------
# attention given indices
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("S", [128, 300])
def test_vs_full_coverage_equals_dense(S):
    """tests/test_vertical_slash_kernel.py:289-303."""
    q, k, v = make_qkv(B=1, H=2, S_q=S, D=64, dtype=torch.float32, seed=S)
    vi = np.broadcast_to(np.arange(S), (1, 2, S))
    si = np.broadcast_to(np.arange(S)[::-1], (1, 2, S))
    sc = O.sparse_scale(64)
    a = O.vertical_slash_from_indices(np32(q), np32(k), np32(v), vi, si, scale=sc)
    b = O.dense_causal(np32(q), np32(k), np32(v), scale=sc)
    assert np.abs(a - b).max() < 1e-12


def test_vs_attention_zero_query_and_rows_bruteforce():
    S, D = 200, 32
    q, k, v = make_qkv(B=1, H=1, S_q=S, D=D, dtype=torch.bfloat16, seed=9)
    g = np.random.default_rng(1)
    vi = np.sort(np.concatenate([np.arange(30), 30 + g.choice(S - 30, 10, replace=False)]))[None, None]
    si = np.sort(np.concatenate([np.arange(50), 50 + g.choice(S - 50, 10, replace=False)]))[::-1][None, None]
    vis = _visible_dual(vi[0, 0], si[0, 0], S)
    vn = np32(v)[0, 0].astype(np.float64)
    qz = np.zeros((1, 1, S, D), np.float32)
    out0 = O.vertical_slash_from_indices(qz, np32(k), np32(v), vi, si)[0, 0]
    for i in (0, 63, 64, 150, S - 1):
        assert np.abs(out0[i] - vn[vis[i]].mean(0)).max() < 1e-12
    out = O.vertical_slash_from_indices(np32(q), np32(k), np32(v), vi, si)[0, 0]
    qn, kn = (np32(t)[0, 0].astype(np.float64) for t in (q, k))
    sc = O.sparse_scale(D)
    for i in (5, 64, 199):
        js = np.nonzero(vis[i])[0]
        lg = qn[i] @ kn[js].T * sc
        p = np.exp(lg - lg.max())
        assert np.abs(out[i] - (p / p.sum()) @ vn[js]).max() < 1e-12
