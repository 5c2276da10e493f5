"""GPU parity of the HIP kernels against the CPU oracle (small sizes).

Bars: block ids bit-exact; attention outputs within 2e-3 max-abs when written
in fp32 (bf16/fp16 inputs, fp32 accumulation); bf16 outputs within 2e-3 plus
one bf16 rounding of the output.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O
from msa_data import dtype_tag, make_qkv, np32

pytestmark = pytest.mark.gpu

TOL = 2e-3


def to_dev(dev, *ts):
    return [t.to(dev) for t in ts]


def assert_close_f32(out: torch.Tensor, ref: np.ndarray, tol=TOL, what=""):
    got = out.detach().float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref).max()
    assert err < tol, f"{what}: max abs err {err:.3e} >= {tol}"
    return err


def assert_close_lowp(out: torch.Tensor, ref: np.ndarray, what=""):
    got = out.detach().float().cpu().numpy().astype(np.float64)
    bound = TOL + np.abs(ref) * 2.0 ** -8
    bad = np.abs(got - ref) > bound
    assert not bad.any(), f"{what}: {bad.sum()} elements outside 2e-3 + bf16 rounding"


# ---------------------------------------------------------------------------
# estimator: bit-exact block ids
# ---------------------------------------------------------------------------
EST_CASES = [
    # (B, H, S_q, S_k, D, topk, dtype, sink)
    (1, 4, 1024, 1024, 96, 4, torch.bfloat16, None),
    (2, 3, 1000, 1000, 96, 3, torch.bfloat16, 8.0),
    (1, 2, 4096 + 17, 4096 + 17, 96, 16, torch.bfloat16, 8.0),
    (1, 2, 2048, 2048, 64, 100, torch.bfloat16, None),
    (1, 2, 2048, 2048, 128, 7, torch.float16, None),
    (1, 4, 640, 640, 96, 1, torch.float16, 8.0),
    (1, 2, 512, 1024, 96, 5, torch.bfloat16, None),
    (1, 2, 100, 700, 96, 3, torch.bfloat16, None),     # chunk with S_k - S_q not a block multiple
    (1, 2, 300, 2000, 96, 100, torch.bfloat16, 8.0),   # top-k clamped to n_kb
]


@pytest.mark.parametrize("case", EST_CASES, ids=[str(c[:6]) + dtype_tag(c[6]) for c in EST_CASES])
def test_estimator_bit_exact(gpu_device, case):
    from minference.ops.block_sparse_kernel import select_block_sparse_topk_indices

    B, H, S_q, S_k, D, topk, dtype, sink = case
    q, k, _ = make_qkv(B, H, S_q, S_k, D, dtype, seed=S_q + topk, sink_scale=sink)
    idx, cnt = select_block_sparse_topk_indices(*to_dev(gpu_device, q, k), topk, return_counts=True)
    ridx, rcnt = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, dtype_tag(dtype))
    got_i = idx.cpu().numpy()
    got_c = cnt.cpu().numpy()
    assert got_i.shape == ridx.shape
    assert np.array_equal(got_c, O.attend_count(ridx, S_q, S_k))
    assert np.array_equal(got_i, ridx), f"{(got_i != ridx).sum()} ids differ"


def test_estimator_long_key_axis(gpu_device):
    """More than 2048 key blocks (S = 200000): the selection keeps its keys
    in the workspace instead of registers; ids bit-exact with the oracle."""
    from minference.ops.block_sparse_kernel import select_block_sparse_topk_indices

    S, topk = 200000, 160
    print(f"[estimator] S={S} topk={topk}", flush=True)
    q, k, _ = make_qkv(1, 2, S, S, 64, torch.bfloat16, seed=11, sink_scale=8.0)
    idx, cnt = select_block_sparse_topk_indices(*to_dev(gpu_device, q, k), topk, return_counts=True)
    ridx, rcnt = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, "bf16")
    got = idx.cpu().numpy()
    assert np.array_equal(cnt.cpu().numpy(), rcnt)
    assert np.array_equal(got, ridx), f"{(got != ridx).sum()} ids differ"


@pytest.mark.parametrize("first,diag", [(False, False), (True, True), (False, True)])
def test_estimator_non_finite_scores(gpu_device, first, diag):
    """NaN and infinite pooled scores (a NaN key, a row of infinite keys, a
    zero query block against it: 0 * inf): NaN ranks above +inf, as
    torch.topk orders it, and forced ids rank above NaN; ids bit-exact with
    the oracle (such rows take the exact fp64 path)."""
    from minference.ops.block_sparse_kernel import select_block_sparse_topk_indices

    S, D, topk = 64 * 24, 96, 4
    q, k, _ = make_qkv(1, 2, S, S, D, torch.bfloat16, seed=5)
    k[0, 0, 64 * 3 + 5, 7] = float("nan")   # block 3 of head 0: NaN in every row's score
    k[0, 1, 64 * 5 + 1, :] = float("inf")   # block 5 of head 1: +-inf or NaN scores
    k[0, 1, 64 * 9 + 2, :48] = float("inf")
    k[0, 1, 64 * 9 + 2, 48:] = float("-inf")
    q[0, 1, 64 * 10:64 * 11] = 0.0          # query block 10 of head 1: 0 * inf
    idx, cnt = select_block_sparse_topk_indices(*to_dev(gpu_device, q, k), topk,
                                                return_counts=True, force_first=first,
                                                force_diag=diag)
    ridx, rcnt = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, "bf16",
                                                    force_first=first, force_diag=diag)
    got = idx.cpu().numpy()
    assert np.array_equal(cnt.cpu().numpy(), rcnt)
    assert np.array_equal(got, ridx), f"{(got != ridx).sum()} ids differ"
    if not first:
        # head 0: the NaN block is selected in every row that sees it (and
        # no forced id outranks it unless the diagonal is forced)
        for bq in range(3, 24):
            assert 3 in got[0, 0, bq, :topk]


def test_estimator_ties_to_lower_id(gpu_device):
    from minference.ops.block_sparse_kernel import select_block_sparse_topk_indices

    S, D = 64 * 40, 96
    blk = torch.randn(64, D)
    k = blk.repeat(40, 1)[None, None].repeat(1, 2, 1, 1).to(torch.bfloat16)
    q = torch.randn(1, 2, S, D).to(torch.bfloat16)
    idx, cnt = select_block_sparse_topk_indices(*to_dev(gpu_device, q, k), 5, return_counts=True)
    idx = idx.cpu().numpy()
    for bq in range(40):
        c = min(5, bq + 1)
        assert list(idx[0, 0, bq, :c]) == list(range(c))


# ---------------------------------------------------------------------------
# stream_llm
# ---------------------------------------------------------------------------
STREAM_CASES = [
    # (n_init, n_local, S_q, S_k, D, dtype)
    (64, 512, 256, 256, 96, torch.bfloat16),      # S_k <= n_local: causal dense
    (4, 8, 9, 9, 96, torch.bfloat16),
    (0, 16, 32, 64, 96, torch.bfloat16),
    (128, 512, 512, 1024, 96, torch.bfloat16),
    (128, 256, 256, 512, 64, torch.float16),
    (400, 128, 128, 512, 128, torch.bfloat16),
    (64, 1, 128, 256, 96, torch.bfloat16),
    (128, 1024, 4096, 4096, 96, torch.bfloat16),
    (100, 800, 3000, 3000, 96, torch.bfloat16),
    (0, 0, 200, 200, 96, torch.bfloat16),         # nothing visible: zeros
]


@pytest.mark.parametrize("case", STREAM_CASES, ids=[str(c[:5]) + dtype_tag(c[5]) for c in STREAM_CASES])
def test_streaming_vs_oracle(gpu_device, case):
    from minference import streaming_forward

    n_init, n_local, s_q, s_k, D, dtype = case
    q, k, v = make_qkv(1, 4, s_q, s_k, D, dtype, seed=42 + s_q)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    streaming_forward(dq, dk, dv, n_init, n_local, out=out32)
    ref = O.streaming_attention(np32(q), np32(k), np32(v), n_init, n_local)
    assert_close_f32(out32, ref, what=f"stream {case}")
    out = streaming_forward(dq, dk, dv, n_init, n_local)
    assert out.dtype == dtype and out.shape == q.shape
    assert_close_lowp(out, ref, what=f"stream lowp {case}")


# ---------------------------------------------------------------------------
# block_sparse
# ---------------------------------------------------------------------------
BLOCK_CASES = [
    # (B, H, S, D, topk, dtype, sink)
    (1, 4, 1024, 96, 4, torch.bfloat16, 8.0),
    (2, 2, 1000, 96, 3, torch.bfloat16, None),
    (1, 2, 2048, 64, 100, torch.bfloat16, None),   # topk > n_blocks: causal dense
    (1, 2, 2048, 128, 8, torch.float16, 8.0),
    (1, 4, 4096, 96, 16, torch.bfloat16, 8.0),
]
BLOCK_CHUNK_CASES = [
    # (S_q, S_k, topk): chunked prefill, the q-frame -inf picks attended
    (100, 700, 3),
    (512, 1024, 5),
    (300, 2000, 100),   # top-k clamped to n_kb: causal dense
    (1000, 4113, 16),
]


@pytest.mark.parametrize("case", BLOCK_CHUNK_CASES, ids=[str(c) for c in BLOCK_CHUNK_CASES])
def test_block_sparse_chunked_vs_oracle(gpu_device, case):
    from minference import block_sparse_attention

    s_q, s_k, topk = case
    q, k, v = make_qkv(1, 3, s_q, s_k, 96, torch.bfloat16, seed=s_q + topk, sink_scale=8.0)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    block_sparse_attention(dq, dk, dv, topk, out=out32)
    idx, _ = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, "bf16")
    ref = O.block_sparse_from_indices(np32(q), np32(k), np32(v), idx)
    assert_close_f32(out32, ref, what=f"block chunk {case}")


@pytest.mark.parametrize("case", BLOCK_CASES, ids=[str(c[:5]) + dtype_tag(c[5]) for c in BLOCK_CASES])
def test_block_sparse_vs_oracle(gpu_device, case):
    from minference import block_sparse_attention

    B, H, S, D, topk, dtype, sink = case
    q, k, v = make_qkv(B, H, S, S, D, dtype, seed=11 + S, sink_scale=sink)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    block_sparse_attention(dq, dk, dv, topk, out=out32)
    idx, _ = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, dtype_tag(dtype))
    ref = O.block_sparse_from_indices(np32(q), np32(k), np32(v), idx)
    assert_close_f32(out32, ref, what=f"block {case}")
    out = block_sparse_attention(dq, dk, dv, topk)
    assert out.dtype == dtype
    assert_close_lowp(out, ref, what=f"block lowp {case}")


def test_block_fixed_indices_with_future_and_duplicates(gpu_device):
    from minference.ops.block_sparse_kernel import block_sparse_attention_with_indices

    B, H, S, D, topk = 1, 3, 1024, 96, 6
    q, k, v = make_qkv(B, H, S, S, D, torch.bfloat16, seed=5)
    n = S // 64
    g = np.random.default_rng(0)
    idx = g.integers(-2, n + 3, size=(B, H, n, topk))  # out of range, future, duplicates
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    block_sparse_attention_with_indices(dq, dk, dv, torch.from_numpy(idx), out=out32)
    ref = O.block_sparse_from_indices(np32(q), np32(k), np32(v), idx)
    assert_close_f32(out32, ref, what="fixed indices")


LARGE_BLOCK_CASES = [
    # (block, B, H, S_q, S_k, D, topk, dtype, sink, force_first, force_diag)
    (128, 1, 3, 1000, 1000, 96, 3, torch.bfloat16, 8.0, False, False),
    (256, 2, 2, 2048 + 17, 2048 + 17, 96, 4, torch.float16, None, False, False),
    (512, 1, 2, 4096, 4096, 128, 2, torch.bfloat16, 8.0, False, False),
    (128, 1, 2, 300, 1100, 96, 3, torch.bfloat16, None, False, False),    # chunk
    (256, 1, 2, 500, 2000, 64, 100, torch.bfloat16, None, False, False),  # top-k clamped
    (128, 1, 2, 1000, 1000, 96, 2, torch.bfloat16, 8.0, True, True),
    (192, 1, 3, 1000, 1000, 96, 3, torch.bfloat16, 8.0, False, False),  # not a power of two
    (320, 1, 2, 700, 1700, 128, 2, torch.float16, None, False, False),   # and chunked
]


@pytest.mark.parametrize("case", LARGE_BLOCK_CASES,
                         ids=[str(c[:7]) + dtype_tag(c[7]) + ("-forced" if c[9] else "")
                              for c in LARGE_BLOCK_CASES])
def test_block_sizes_above_64(gpu_device, case):
    """Selector ids and counts bit-exact at blocks of 128 to 512 tokens, and the
    attention over those blocks within the bars of the 64-token path."""
    from minference import block_sparse_attention
    from minference.ops.block_sparse_kernel import select_block_sparse_topk_indices

    block, B, H, S_q, S_k, D, topk, dtype, sink, first, diag = case
    q, k, v = make_qkv(B, H, S_q, S_k, D, dtype, seed=block + S_q, sink_scale=sink)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    idx, cnt = select_block_sparse_topk_indices(dq, dk, topk, block, return_counts=True,
                                                force_first=first, force_diag=diag)
    ridx, rcnt = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, dtype_tag(dtype),
                                                    block=block, force_first=first,
                                                    force_diag=diag)
    got_i, got_c = idx.cpu().numpy(), cnt.cpu().numpy()
    assert got_i.shape == ridx.shape
    assert np.array_equal(got_i, ridx), f"{(got_i != ridx).sum()} ids differ"
    assert np.array_equal(got_c, O.attend_count(ridx, S_q, S_k, block))
    ref = O.block_sparse_from_indices(np32(q), np32(k), np32(v), ridx, block=block)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    block_sparse_attention(dq, dk, dv, topk, block, out=out32, force_first=first,
                           force_diag=diag)
    assert_close_f32(out32, ref, what=f"block {block} {case[1:7]}")
    out = block_sparse_attention(dq, dk, dv, topk, block, force_first=first, force_diag=diag)
    assert out.dtype == dtype
    assert_close_lowp(out, ref, what=f"block {block} lowp {case[1:7]}")


@pytest.mark.parametrize("block,s_q,s_k", [(128, 1000, 1000), (256, 300, 1300), (512, 1100, 1100),
                                           (192, 900, 900)])
def test_block_fixed_indices_large_blocks(gpu_device, block, s_q, s_k):
    """Fixed ids of 128- to 512-token blocks: out of range, negative, future
    and repeated ids; chunked rows (S_q < S_k)."""
    from minference.ops.block_sparse_kernel import block_sparse_attention_with_indices

    B, H, D, topk = 1, 3, 96, 4
    q, k, v = make_qkv(B, H, s_q, s_k, D, torch.bfloat16, seed=block + s_k)
    n_bq, n_bk = -(-s_q // block), -(-s_k // block)
    g = np.random.default_rng(block)
    idx = g.integers(-2, n_bk + 2, size=(B, H, n_bq, topk))
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    block_sparse_attention_with_indices(dq, dk, dv, torch.from_numpy(idx), block, out=out32)
    ref = O.block_sparse_from_indices(np32(q), np32(k), np32(v), idx, block=block)
    assert_close_f32(out32, ref, what=f"fixed indices block {block}")


# ---------------------------------------------------------------------------
# dense
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("s_q,s_k,D,dtype", [(1024, 1024, 96, torch.bfloat16),
                                             (300, 700, 96, torch.bfloat16),
                                             (1, 500, 96, torch.bfloat16),
                                             (512, 512, 128, torch.float16),
                                             (2000, 2000, 64, torch.bfloat16)])
def test_dense_vs_oracle(gpu_device, s_q, s_k, D, dtype):
    from minference import dense_attention

    q, k, v = make_qkv(1, 3, s_q, s_k, D, dtype, seed=s_q)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    dense_attention(dq, dk, dv, out=out32)
    ref = O.dense_causal(np32(q), np32(k), np32(v))
    assert_close_f32(out32, ref, what="dense")


@pytest.mark.parametrize("s_q,s_k,D,dtype", [(256, 256, 96, torch.bfloat16),
                                              (100, 700, 96, torch.bfloat16),
                                              (700, 100, 64, torch.float16),
                                              (1000, 1000, 128, torch.bfloat16),
                                              (65, 3000, 96, torch.bfloat16)])
def test_dense_noncausal_vs_oracle(gpu_device, s_q, s_k, D, dtype):
    """dense_attention(causal=False) (reference backend_npu/attention.py:221-230):
    every key visible to every query, S_q > S_k included."""
    from minference import dense_attention

    print(f"[dense non-causal] {s_q} {s_k} {D} {dtype}", flush=True)
    q, k, v = make_qkv(1, 3, s_q, s_k, D, dtype, seed=s_q + s_k, use_rope=False)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    dense_attention(dq, dk, dv, causal=False, out=out32)
    ref = O.dense_causal(np32(q), np32(k), np32(v), causal=False)
    assert_close_f32(out32, ref, what="dense non-causal")
    out = dense_attention(dq, dk, dv, causal=False)
    assert out.dtype == dtype
    assert_close_lowp(out, ref, what="dense non-causal lowp")


FORCED_CASES = [
    # (S, D, topk, dtype, force_first, force_diag)
    (4096 + 17, 96, 16, torch.bfloat16, True, True),
    (4096, 96, 100, torch.bfloat16, True, True),
    (2048, 128, 7, torch.float16, False, True),
    (3000, 64, 4, torch.bfloat16, True, False),
    (1024, 96, 1, torch.bfloat16, True, True),
    (1024, 96, 2, torch.bfloat16, False, True),
]


@pytest.mark.parametrize("case", FORCED_CASES, ids=[str(c) for c in FORCED_CASES])
def test_estimator_forced_bit_exact(gpu_device, case):
    """The selector option that always keeps block 0 and/or the diagonal
    block (inside the top-k): ids bit-exact with the oracle."""
    from minference.ops.block_sparse_kernel import select_block_sparse_topk_indices

    S, D, topk, dtype, first, diag = case
    q, k, _ = make_qkv(1, 4, S, S, D, dtype, seed=S + topk, sink_scale=8.0)
    idx, cnt = select_block_sparse_topk_indices(*to_dev(gpu_device, q, k), topk,
                                                return_counts=True, force_first=first,
                                                force_diag=diag)
    ridx, rcnt = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, dtype_tag(dtype),
                                                    force_first=first, force_diag=diag)
    got = idx.cpu().numpy()
    assert np.array_equal(cnt.cpu().numpy(), rcnt)
    assert np.array_equal(got, ridx), f"{(got != ridx).sum()} ids differ"
    nb = ridx.shape[-2]
    for bq in range(nb):
        c = rcnt[0, 0, bq]
        row = set(got[0, 0, bq, :c].tolist())
        if first:
            assert 0 in row
        if diag and not (first and c == 1 and bq > 0):
            assert bq in row


@pytest.mark.parametrize("factor", [4.0, 12.0, 40.0])
@pytest.mark.parametrize("kind", ["dense", "stream", "block"])
def test_late_outlier_keys(gpu_device, kind, factor):
    """Keys scaled by `factor` in the middle of the sequence make a row's max
    logit jump after its first tiles: by a few units (P stays below 2^8, no
    rescale), past that slack, or far enough that P taken with the stale
    maximum would overflow fp16 and fp32; the last two take the rare path
    (scores recomputed, O and the row sums rescaled) mid-item."""
    from minference import block_sparse_attention, dense_attention, streaming_forward

    S, H, D = 2048, 2, 96
    q, k, v = make_qkv(1, H, S, S, D, torch.bfloat16, seed=int(factor))
    k = k.float()
    for j in (1500, 1501, 1777):
        k[:, :, j] *= factor
    k = k.to(torch.bfloat16)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    qn, kn, vn = np32(q), np32(k), np32(v)
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    if kind == "dense":
        dense_attention(dq, dk, dv, out=out32)
        ref = O.dense_causal(qn, kn, vn)
    elif kind == "stream":
        streaming_forward(dq, dk, dv, 64, 1024, out=out32)
        ref = O.streaming_attention(qn, kn, vn, 64, 1024)
    else:
        block_sparse_attention(dq, dk, dv, 6, out=out32)
        idx, _ = O.select_block_sparse_topk_indices(qn, kn, 6, "bf16")
        ref = O.block_sparse_from_indices(qn, kn, vn, idx)
    assert_close_f32(out32, ref, what=f"{kind} x{factor}")


# ---------------------------------------------------------------------------
# decode: one query row against the whole cache
# ---------------------------------------------------------------------------
DECODE_CASES = [
    # (B, H, H_kv, S_k, D, dtype)
    (1, 4, 4, 1, 96, torch.bfloat16),
    (1, 4, 4, 63, 96, torch.bfloat16),
    (2, 3, 3, 1000, 96, torch.bfloat16),
    (1, 8, 2, 4096 + 17, 96, torch.bfloat16),
    (1, 4, 4, 2048, 64, torch.float16),
    (1, 2, 2, 3000, 128, torch.bfloat16),
    (1, 2, 2, 70000, 96, torch.bfloat16),
]


def _decode_inputs(B, H, Hkv, S, D, dtype, seed):
    q, _, _ = make_qkv(B, H, 1, S, D, dtype, seed=seed)             # RoPE at position S-1
    _, k, v = make_qkv(B, Hkv, S, S, D, dtype, seed=seed + 1, sink_scale=8.0)
    return q, k, v


@pytest.mark.parametrize("case", DECODE_CASES, ids=[str(c[:5]) + dtype_tag(c[5]) for c in DECODE_CASES])
def test_decode_vs_oracle(gpu_device, case):
    from minference.backend.attention import decode_dense

    B, H, Hkv, S, D, dtype = case
    q, k, v = _decode_inputs(B, H, Hkv, S, D, dtype, seed=S)
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    ref = O.dense_causal(np32(q), np32(k), np32(v))  # the single row sees every key
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    decode_dense(dq, dk, dv, out=out32)
    assert_close_f32(out32, ref, what=f"decode {case}")
    out = decode_dense(dq, dk, dv, scale=0.05)
    assert out.dtype == dtype
    assert_close_lowp(out, O.dense_causal(np32(q), np32(k), np32(v), scale=0.05), what=f"decode lowp {case}")


def test_decode_strided_cache_view(gpu_device):
    """The cache as a slice of a preallocated [B, S_max, H, D] buffer."""
    from minference.backend.attention import decode_dense

    B, H, S, S_max, D = 2, 4, 777, 1024, 96
    q, k, v = _decode_inputs(B, H, H, S, D, torch.bfloat16, seed=5)
    kbuf = torch.zeros(B, S_max, H, D, dtype=torch.bfloat16)
    vbuf = torch.zeros(B, S_max, H, D, dtype=torch.bfloat16)
    kbuf[:, :S] = k.transpose(1, 2)
    vbuf[:, :S] = v.transpose(1, 2)
    dkb, dvb = to_dev(gpu_device, kbuf, vbuf)
    dk, dv = dkb.transpose(1, 2)[:, :, :S], dvb.transpose(1, 2)[:, :, :S]
    assert dk.stride(2) == H * D
    out32 = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    decode_dense(q.to(gpu_device), dk, dv, out=out32)
    assert_close_f32(out32, O.dense_causal(np32(q), np32(k), np32(v)), what="decode strided")


# ---------------------------------------------------------------------------
# one mixed layer through the dispatcher plan; strided (HF-like) views; GQA
# ---------------------------------------------------------------------------
def _mixed_patterns(H):
    kinds = [("stream_llm", 64, 256), ("block_sparse", 5, 0), ("dense", 0, 0),
             ("block_sparse", 2, 0), ("stream_llm", 0, 128), ("block_sparse", 100, 0)]
    return {h: list(kinds[h % len(kinds)]) + [1.0] for h in range(H)}


MIXED_SHAPES = [
    # (B, H, H_kv, S_q, S_k, D, dtype)
    (2, 8, 8, 777, 777, 96, torch.bfloat16),     # batch 2, S not a multiple of 64
    (1, 6, 1, 1000, 1000, 64, torch.float16),    # one kv head (MQA), D 64, fp16
    (1, 4, 2, 640, 640, 128, torch.bfloat16),    # D 128, GQA
    (2, 8, 4, 300, 1324, 96, torch.bfloat16),    # chunked prefill, batch 2
    (1, 8, 8, 130, 4000, 96, torch.float16),     # short chunk after a long cache
    (1, 4, 2, 700, 700, 256, torch.bfloat16),    # D 256 (the row-split kernel), GQA
    (1, 6, 3, 300, 1100, 256, torch.float16),    # D 256, chunked prefill, fp16
    (1, 4, 2, 500, 500, 512, torch.bfloat16),    # D 512 (one wave per SIMD)
]


@pytest.mark.parametrize("case", MIXED_SHAPES,
                         ids=[str(c[:6]) + dtype_tag(c[6]) for c in MIXED_SHAPES])
def test_mixed_layer_shapes(gpu_device, case):
    """The patched layer's mixed dispatch (stream / block with its estimator /
    dense in one launch) over batch, GQA / MQA, head dims, fp16 and
    chunked prefill, against the oracle's per-head layer."""
    from minference.modules.minference_forward import build_layer_plan, run_layer_attention

    B, H, Hkv, S_q, S_k, D, dtype = case
    print(f"[mixed] case {case}", flush=True)
    pats = _mixed_patterns(H)
    q, k, v = make_qkv(B, H, S_q, S_k, D, dtype, seed=S_q + 7 * H, sink_scale=8.0)
    k, v = k[:, :Hkv].contiguous(), v[:, :Hkv].contiguous()
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    plan = build_layer_plan(pats, H, D, S_k)
    out = torch.empty((B, H, S_q, D), dtype=torch.float32, device=gpu_device)
    run_layer_attention(dq, dk, dv, plan, out)
    rep = H // Hkv
    ref, _ = O.layer_attention(np32(q), np.repeat(np32(k), rep, axis=1),
                               np.repeat(np32(v), rep, axis=1), [pats[h] for h in range(H)],
                               dtype_tag(dtype))
    assert_close_f32(out, ref, what=f"mixed layer {case}")


@pytest.mark.parametrize("S,H,H_kv", [(1024, 8, 8), (1000, 8, 2), (2048, 16, 16)])
def test_mixed_layer_strided_views(gpu_device, S, H, H_kv):
    from minference.modules.minference_forward import build_layer_plan, run_layer_attention

    D = 96
    pats = _mixed_patterns(H)
    q, k, v = make_qkv(1, H, S, S, D, torch.bfloat16, seed=S + H, sink_scale=8.0)
    k, v = k[:, :H_kv].contiguous(), v[:, :H_kv].contiguous()
    # fused [B, S, (H + 2 H_kv) D] buffer and BNSD views into it, as HF's qkv_proj split
    fused = torch.cat([q.transpose(1, 2).reshape(1, S, H * D),
                       k.transpose(1, 2).reshape(1, S, H_kv * D),
                       v.transpose(1, 2).reshape(1, S, H_kv * D)], dim=-1).to(gpu_device)
    dq = fused[..., :H * D].view(1, S, H, D).transpose(1, 2)
    dk = fused[..., H * D:(H + H_kv) * D].view(1, S, H_kv, D).transpose(1, 2)
    dv = fused[..., (H + H_kv) * D:].view(1, S, H_kv, D).transpose(1, 2)
    plan = build_layer_plan(pats, H, D, S)
    out_bshd = torch.empty((1, S, H, D), dtype=torch.float32, device=gpu_device)
    run_layer_attention(dq, dk, dv, plan, out_bshd.transpose(1, 2))
    rep = H // H_kv
    kr = np.repeat(np32(k), rep, axis=1)
    vr = np.repeat(np32(v), rep, axis=1)
    ref, _ = O.layer_attention(np32(q), kr, vr, [pats[h] for h in range(H)], "bf16")
    assert_close_f32(out_bshd.transpose(1, 2), ref, what=f"mixed layer S={S} H={H} Hkv={H_kv}")


@pytest.mark.parametrize("S", [200, 1000])
@pytest.mark.parametrize("which", ["q", "k"])
def test_mixed_layer_strided_rows(gpu_device, S, which):
    """q or k views with unusual row strides are read as the tensor the view
    describes, against the oracle on the materialised view: an expanded view
    (stride 0, every row the same) and overlapping rows (stride D/2; for k
    both take the staged-K path), and padded rows (stride D + 40; k read in
    place with a row stride above D)."""
    from minference.modules.minference_forward import build_layer_plan, run_layer_attention

    H, D = 4, 96
    pats = _mixed_patterns(H)
    q, k, v = make_qkv(1, H, S, S, D, torch.bfloat16, seed=S, sink_scale=8.0)
    plan = build_layer_plan(pats, H, D, S)
    src = q if which == "q" else k
    base = src[:, :, :1].to(gpu_device)
    flat = src.reshape(1, H, -1)[:, :, :(S + 1) * D // 2].contiguous().to(gpu_device)
    wide = torch.zeros((1, H, S, D + 40), dtype=src.dtype)
    wide[..., :D] = src
    views = {
        "expanded": base.expand(1, H, S, D),
        "overlapping": flat.as_strided((1, H, S, D), (H * flat.shape[-1], flat.shape[-1], D // 2, 1)),
        "padded": wide.to(gpu_device)[..., :D],
    }
    for name, dx in views.items():
        print(f"[strided rows] {which} {name} S={S}", flush=True)
        dq = dx if which == "q" else q.to(gpu_device)
        dk = dx if which == "k" else k.to(gpu_device)
        out = torch.empty((1, H, S, D), dtype=torch.float32, device=gpu_device)
        run_layer_attention(dq, dk, v.to(gpu_device), plan, out)
        ref, _ = O.layer_attention(np32(dq.cpu().contiguous()), np32(dk.cpu().contiguous()),
                                   np32(v), [pats[h] for h in range(H)], "bf16")
        assert_close_f32(out, ref, what=f"{name} {which} rows S={S}")


# ---------------------------------------------------------------------------
# float32 inputs
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rng", ["fp16", "bf16"])
def test_float32_inputs(gpu_device, rng):
    """float32 q/k/v (the reference's CPU paths compute them in fp32,
    streaming_kernel_npu.py:138-144, block_sparse_kernel_npu.py:340-348) run
    as their on-device roundings to fp16, or to bf16 when a finite value
    exceeds fp16's range, with a float32 output: every op equals the same
    call on the explicitly rounded inputs, bit for bit, and the stream op
    stays within the fp32-output tolerance of the oracle on those roundings.
    (Against the oracle on the float32 inputs themselves the fp16 rounding of
    q and k moves this case's outputs by up to about 8e-3: the sink keys are
    scaled by 8, so their logits carry the larger rounding.)"""
    from minference import block_sparse_attention, dense_attention, streaming_forward
    from minference.backend.attention import decode_dense
    from minference.ops.block_sparse_kernel import (block_sparse_attention_with_indices,
                                                    select_block_sparse_topk_indices)
    from minference.ops.vertical_slash_kernel import (vertical_and_slash_attention,
                                                      vertical_and_slash_estimate,
                                                      vertical_slash_sparse_attention)

    print(f"[float32 inputs] {rng}", flush=True)
    B, H, S, D = 1, 4, 700, 96
    q, k, v = make_qkv(B, H, S, S, D, torch.float32, seed=21, sink_scale=8.0)
    if rng == "bf16":
        v = v.clone()
        v[0, 1, 5, 3] = 1.0e5
    dt = torch.float16 if rng == "fp16" else torch.bfloat16
    dq, dk, dv = to_dev(gpu_device, q, k, v)
    rq, rk, rv = (t.to(dt) for t in (dq, dk, dv))
    vi = torch.arange(0, S, 9).expand(B, H, -1)
    si = torch.arange(198, -1, -3).expand(B, H, -1)
    calls = {
        "stream": lambda a, b, c, **o: streaming_forward(a, b, c, 64, 256, **o),
        "block": lambda a, b, c, **o: block_sparse_attention(a, b, c, 5, **o),
        "dense": lambda a, b, c, **o: dense_attention(a, b, c, **o),
        "decode": lambda a, b, c, **o: decode_dense(a[:, :, -1:], b, c, **o),
        "vs": lambda a, b, c, **o: vertical_slash_sparse_attention(a, b, c, vi, si, **o),
        "block ids": lambda a, b, c, **o: block_sparse_attention_with_indices(a, b, c, bi, **o),
        "vs layer": lambda a, b, c, **o: vertical_and_slash_attention(a, b, c, 100, 200, **o),
    }
    bi = torch.randint(0, S // 64 + 1, (B, H, S // 64 + 1, 4), generator=torch.Generator().manual_seed(3))
    for name, call in calls.items():
        got = call(dq, dk, dv)
        assert got.dtype == torch.float32, name
        ref = torch.empty(got.shape, dtype=torch.float32, device=gpu_device)
        call(rq, rk, rv, out=ref)
        assert torch.equal(got, ref), name
    # the estimators see q and k only, which fit fp16 in both cases
    assert torch.equal(select_block_sparse_topk_indices(dq, dk, 5),
                       select_block_sparse_topk_indices(dq.half(), dk.half(), 5))
    for a, b in zip(vertical_and_slash_estimate(dq, dk, 100, 200),
                    vertical_and_slash_estimate(dq.half(), dk.half(), 100, 200)):
        assert torch.equal(a, b)
    if rng == "fp16":
        ref = O.streaming_attention(np32(rq), np32(rk), np32(rv), 64, 256)
        assert_close_f32(streaming_forward(dq, dk, dv, 64, 256), ref, what="float32 stream")

    # a padded head dim (200 -> 256) and a block of 128 tokens, same rule
    q2, k2, v2 = make_qkv(1, 2, 500, 500, 200, torch.float32, seed=22, sink_scale=8.0)
    d2 = to_dev(gpu_device, q2, k2, v2)
    r2 = [t.to(torch.float16) for t in d2]
    for name, call in {
        "stream D200": lambda a, b, c, **o: streaming_forward(a, b, c, 32, 128, **o),
        "block D200 bs128": lambda a, b, c, **o: block_sparse_attention(a, b, c, 2, 128, **o),
    }.items():
        got = call(*d2)
        assert got.dtype == torch.float32 and got.shape == q2.shape, name
        want = call(*r2, out=torch.empty(q2.shape, dtype=torch.float32, device=gpu_device))
        assert torch.equal(got, want), f"{name}: differs from the call on rounded inputs"
