"""Census: the oracle's vertical_and_slash estimator against the reference's
own torch steps at full length (CPU).

The reference estimator (minference/modules/minference_forward.py:140-165) is
run here as the torch calls it makes, on bf16 Q/K: the bf16 ``matmul`` of the
last 64 rows with K^T divided by ``math.sqrt(D)``, the last-rows causal
``-inf`` mask, ``softmax(dtype=float32)``, fp32 column sums, fp32 diagonal
sums over the zero-padded strided view (sum_all_diagonal_matrix, :124-137),
the forced +inf columns / diagonals, ``topk``.  The oracle (and the GPU
estimator, bit exact with it) forms the logits from the exact dot product,
takes the softmax and the sums in fp64 and rounds each sum once to fp32.

Two checks per head:
  * logits: every reference logit x_r equals the oracle's x_o up to what the
    reference's fp32 accumulation can move it: |x_r - x_o| <=
    (gamma_96 sum_d |q_d k_d| + ulp16(a)) / sqrt(D) + ulp16(x), with a the
    matmul output and ulp16 one unit in the last place of the 16-bit type;
  * selections: where the selected sets differ, every id the oracle keeps
    and the reference drops (a) and the converse (b) form a near-tie:
    V_o(a) - V_o(b) <= B(a) + B(b), B(j) the bound on |V_r(j) - V_o(j)|
    that follows from the measured logit differences Delta (a softmax
    weight moves by at most the factor exp(|Delta_ij| + max_j' |Delta_ij'|)),
    the fp32 softmax (exp to 2 ulp, x - m to one rounding, a sum of S terms
    to gamma_S, the normalisation to 2 roundings) and the fp32 sums of 64
    terms (gamma_64), plus the oracle's own rounding to fp32.

Shapes: S = 65536 and 131072 (the bench's vs64k length and the kernel's
maximum), the (vertical, slash) sizes of the Phi-3 pattern file's three
kinds of VS heads, RoPE'd N(0, 1) Q/K with K rows 0-3 x8 from the tests'
generator recipe."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O
from msa_data import rope

U = 2.0 ** -24


def _gamma(n: int) -> float:
    return n * U / (1 - n * U)


def _qk(S, D, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    out = []
    for name in "qk":
        x = torch.randn(1, 1, S, D, generator=g)
        for s0 in range(0, S, 8192):
            x[:, :, s0:s0 + 8192] = rope(x[:, :, s0:s0 + 8192], offset=s0)
        if name == "k":
            x[:, :, :4] *= 8.0
        out.append(x.to(torch.bfloat16))
    return out


def _reference_steps(q, k, vsz, ssz):
    """The reference's estimator steps as torch calls (:143-164) on one head:
    returns (logits [n, S] as fp64, fp32 vertical sums, fp32 diagonal sums,
    vertical ids, slash ids)."""
    S, D = q.shape[-2], q.shape[-1]
    n = min(64, S)
    nv, ns = min(S, max(vsz, 30)), min(S, max(ssz, 50))
    qk = torch.matmul(q[:, :, -n:, :], k.transpose(-2, -1)) / math.sqrt(D)
    keep = torch.arange(n)[:, None] >= torch.arange(n)[None, :]
    qk[:, :, :, -n:] = torch.where(keep, qk[:, :, :, -n:], float("-inf"))
    x = qk[0, 0].double()
    p = torch.softmax(qk, dim=-1, dtype=torch.float32)
    vert = p.sum(-2, keepdim=True)
    # diagonal sums: zero-pad n columns on both sides, view row i shifted by
    # i + 1 columns, sum over the rows, drop the first and the last n - 1
    pad = torch.zeros(1, 1, n, n, dtype=p.dtype)
    wide = torch.cat((pad, p, pad), -1).contiguous()
    w = wide.shape[-1]
    diag = wide.as_strided((1, 1, n, n + S), (n * w, n * w, w + 1, 1)).sum(2)[..., 1:]
    diag = diag[..., : -n + 1] if n > 1 else diag
    vsum, dsum = vert[0, 0, 0].clone(), diag[0, 0].clone()
    vert[..., :30] = torch.inf
    diag[..., -100:] = torch.inf
    v_idx = torch.topk(vert, nv, dim=-1).indices.reshape(-1).sort().values
    s_idx = ((S - 1) - torch.topk(diag, ns, dim=-1).indices.reshape(-1)).sort(descending=True).values
    return x.numpy(), vsum.double().numpy(), dsum.double().numpy(), v_idx.numpy(), s_idx.numpy()


def _ulp16(x: np.ndarray) -> np.ndarray:
    """One bf16 unit in the last place at |x| (8 significant bits), taken
    in the next binade up when |x| lies within 2^-6 of it (two values that
    round differently may sit on either side of a power of two)."""
    e = np.floor(np.log2(np.maximum(np.abs(x) * (1 + 2.0 ** -6), 2.0 ** -126)))
    return 2.0 ** (e - 7)


@pytest.mark.parametrize("S", [65536, 131072])
@pytest.mark.parametrize("vsz,ssz", [(3500, 100), (1000, 6096), (100, 750)],
                         ids=["v3500-s100", "v1000-s6096", "v100-s750"])
def test_vs_estimator_census(S, vsz, ssz):
    D = 96
    q, k = _qk(S, D, seed=S // 1024 + vsz)
    xr, vr, dr, ref_v, ref_s = _reference_steps(q, k, vsz, ssz)
    qn, kn = q[0, 0].float().numpy(), k[0, 0].float().numpy()
    n = min(64, S)

    # logits: the reference's differ from the oracle's only within the
    # fp32 accumulation bound of the 96-term bf16 dot products
    xo = O.vs_logits(qn, kn, "bf16")
    assert np.array_equal(np.isinf(xo), np.isinf(xr))
    fin = np.isfinite(xo)
    prod_abs = np.abs(qn[S - n:].astype(np.float64)) @ np.abs(kn.astype(np.float64)).T
    a = xo * math.sqrt(D)
    lim = (_gamma(D) * prod_abs + _ulp16(a)) / math.sqrt(D) + _ulp16(xo)
    with np.errstate(invalid="ignore"):                        # -inf - -inf where masked
        delta = np.where(fin, np.abs(np.where(fin, xr - xo, 0.0)), 0.0)
    assert (delta <= np.where(fin, lim, 0.0)).all(), float((delta - lim)[fin].max())
    n_logits = int((delta > 0).sum())

    # selections
    ov, os_ = O.vs_estimate(qn[None, None], kn[None, None], vsz, ssz, "bf16")
    ov, os_ = ov[0, 0], os_[0, 0]
    p = O.vs_probs(xo)
    vo = p.sum(axis=0)
    do = O.vs_diagonal_sums(p)
    dmax = delta.max(axis=1, keepdims=True)
    m = np.where(np.isfinite(xr), xr, -np.inf).max(axis=1, keepdims=True)
    with np.errstate(invalid="ignore"):
        eps_sm = 3 * U + U * np.where(fin, np.abs(xr - m), 0.0) + _gamma(S) + 2 * U
    hi = p * np.exp(delta + dmax) * (1 + eps_sm)              # bound on the reference's weight
    move = p * (np.exp(delta + dmax) * (1 + eps_sm) - 1)       # bound on |p_r - p|
    bound_v = move.sum(axis=0) + _gamma(n) * hi.sum(axis=0) + 2 * U * vo
    bound_d = O.vs_diagonal_sums(move) + _gamma(n) * O.vs_diagonal_sums(hi) + 2 * U * do

    worst = 0.0
    diffs = 0
    for got, ref, val, bnd, forced in ((ov, ref_v, vo, bound_v, set(range(30))),
                                       (S - 1 - os_, S - 1 - ref_s, do, bound_d,
                                        set(range(max(0, S - 100), S)))):
        only_o = sorted(set(got.tolist()) - set(ref.tolist()))
        only_r = sorted(set(ref.tolist()) - set(got.tolist()))
        assert len(only_o) == len(only_r)
        assert not (forced & set(only_o)) and not (forced & set(only_r))
        diffs += len(only_o)
        for x in only_o:
            for y in only_r:
                gap = val[x] - val[y]          # the oracle ranks x above y
                slack = bnd[x] + bnd[y]
                worst = max(worst, gap / slack)
                assert gap <= slack, (x, y, gap, slack)
    # the reference's own sums lie inside the bound around the oracle's
    assert (np.abs(vr[30:] - vo[30:]) <= bound_v[30:]).all()
    assert (np.abs(dr[: S - 100] - do[: S - 100]) <= bound_d[: S - 100]).all()
    print(f"[vs census] S={S} ({vsz}, {ssz}): {n_logits} of {int(fin.sum())} logits differ "
          f"(all within the accumulation bound); {diffs} ids differ; worst gap / bound "
          f"{worst:.3f}")
