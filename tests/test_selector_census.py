"""Census: the oracle's block selection against the reference's own selector
arithmetic, at the benchmark shapes (CPU).

The reference selector (minference/ops/block_sparse_kernel_npu.py:240-263) is
run here as the torch ops it calls: bf16 ``mean(dim=3)`` pooling, ``.to(fp32)``,
fp32 ``matmul`` times 128**-0.5 (the padded-D scale), the block-causal
``-inf`` mask, ``topk`` and ``sort``.  The oracle (and the GPU estimator, bit
exact with it) ranks by the correctly rounded fp32 score, ties to the lower
id; the reference's fp32 sgemm rounds its 96-term sums in some order.  They
can only disagree where two candidates' exact scores are closer than the
sgemm's error bound.  This test counts the rows where the selected sets
differ and proves each difference is such a near-tie: for every id the oracle
keeps and the reference drops (a) and the converse (b), the exact (fp64)
scores satisfy |s(a) - s(b)| <= err(a) + err(b) + 4 ulp, with
err(x) = gamma_96 * sum_d |q_d k_d| the standard bound of a 96-term fp32 dot
product in any summation order (gamma_n = n u / (1 - n u), u = 2^-24).

Shapes: BASELINE config 2 (S = 16384, 32 heads, top-100) and the benchmark's
64K headline (S = 65536, 16 block heads, top-100), N(0,1) Q/K with RoPE and K
rows 0-3 x8, generated on the CPU with the tests' recipe."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from msa_data import rope

U = 2.0 ** -24


def _qk(H, S, D, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    out = []
    for name in "qk":
        x = torch.randn(1, H, S, D, generator=g)
        for s0 in range(0, S, 8192):
            x[:, :, s0:s0 + 8192] = rope(x[:, :, s0:s0 + 8192], offset=s0)
        if name == "k":
            x[:, :, :4] *= 8.0
        out.append(x.to(torch.bfloat16))
    return out


def _reference_selector(q, k, topk, scale):
    """The reference's steps as torch calls (block_sparse_kernel_npu.py:249-263)."""
    B, H, S, D = q.shape
    nb = S // 64
    qp = q.reshape(B, H, nb, 64, D).mean(dim=3).to(torch.float32)
    kp = k.reshape(B, H, nb, 64, D).mean(dim=3).to(torch.float32)
    sc = torch.matmul(qp, kp.transpose(-2, -1)) * scale
    causal = torch.arange(nb)[:, None] >= torch.arange(nb)[None, :]
    sc.masked_fill_(~causal[None, None], float("-inf"))
    return torch.topk(sc, min(topk, nb), dim=-1).indices.sort(dim=-1).values, qp, kp


@pytest.mark.parametrize("H,S,topk,seed", [(32, 16384, 100, 2), (16, 65536, 100, 0)],
                         ids=["cfg2_16k", "headline_64k"])
def test_selector_census(H, S, topk, seed):
    D = 96
    scale = 128 ** -0.5
    q, k = _qk(H, S, D, seed)
    ref, qp, kp = _reference_selector(q, k, topk, scale)
    ref = ref.numpy()
    qn, kn = q.float().numpy(), k.float().numpy()
    idx, cnt = O.select_block_sparse_topk_indices(qn, kn, topk, "bf16", scale)
    # the oracle's pooling is torch's bf16 mean, bit for bit
    assert np.array_equal(O.pool_blocks(qn, "bf16"), qp.numpy())
    assert np.array_equal(O.pool_blocks(kn, "bf16"), kp.numpy())
    qd, kd = qp.numpy().astype(np.float64), kp.numpy().astype(np.float64)
    nb = S // 64
    gamma = 96 * U / (1 - 96 * U)
    rows_diff = ids_diff = 0
    worst = 0.0
    for h in range(H):
        for bq in range(topk, nb):  # rows with fewer causal blocks than top-k agree trivially
            a = set(idx[0, h, bq, :cnt[0, h, bq]].tolist())
            b = set(ref[0, h, bq].tolist())
            if a == b:
                continue
            rows_diff += 1
            only_a, only_b = sorted(a - b), sorted(b - a)
            ids_diff += len(only_a)
            assert len(only_a) == len(only_b)
            prod = qd[0, h, bq][None, :] * kd[0, h]
            exact = prod.sum(-1) * scale
            err = gamma * np.abs(prod).sum(-1) * scale
            for x in only_a:
                for y in only_b:
                    gap = abs(exact[x] - exact[y])
                    slack = err[x] + err[y] + 4 * U * max(abs(exact[x]), abs(exact[y]))
                    worst = max(worst, gap / slack)
                    assert gap <= slack, (h, bq, x, y, gap, slack)
    print(f"[census] H={H} S={S} top-{topk}: {rows_diff} of {H * (nb - topk)} rows differ "
          f"({ids_diff} ids), worst gap / bound = {worst:.3f}")
