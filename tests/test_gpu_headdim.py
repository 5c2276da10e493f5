"""GPU parity of the op layer at head dims the kernels are not built for.

The reference pads head_dim to 16/32/64/128/256/512 before its kernels
(minference/ops/streaming_kernel_npu.py:377-381,
minference/ops/block_sparse_kernel_npu.py:651-656) and cuts the output back.
This build pads q, k and v with zeros to the next built size (64, 96, 128,
256, 512),
which changes no dot product and no pooled mean, and keeps the scale of the
original head_dim by the reference's rule: (next allowed size)^-0.5 for
stream_llm / block_sparse, 1/sqrt(D) for dense and decode.  Checked against
the oracle on the unpadded inputs: block ids bit-exact, outputs within 2e-3
(fp32 outputs).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from msa_data import make_qkv, np32

pytestmark = pytest.mark.gpu

TOL = 2e-3
DIMS = (40, 80, 112, 160, 200, 256, 320, 512)


def _err(out, ref):
    got = out.detach().float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    return float(np.abs(got - ref).max())


@pytest.mark.parametrize("D", DIMS)
def test_padded_head_dim_ops(gpu_device, D):
    from minference import block_sparse_attention, dense_attention, streaming_forward
    from minference.backend.attention import decode_dense
    from minference.ops.block_sparse_kernel import select_block_sparse_topk_indices

    print(f"[headdim] D={D}", flush=True)
    S = 1000
    q, k, v = make_qkv(1, 3, S, S, D, torch.bfloat16, seed=70 + D, sink_scale=8.0)
    dq, dk, dv = (t.to(gpu_device) for t in (q, k, v))
    qn, kn, vn = np32(q), np32(k), np32(v)

    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    streaming_forward(dq, dk, dv, 64, 256, out=out)
    assert _err(out, O.streaming_attention(qn, kn, vn, 64, 256)) < TOL

    ids = select_block_sparse_topk_indices(dq, dk, 4).cpu().numpy()
    ref_ids, _ = O.select_block_sparse_topk_indices(qn, kn, 4, "bf16")
    assert np.array_equal(ids, ref_ids)
    block_sparse_attention(dq, dk, dv, 4, out=out)
    assert _err(out, O.block_sparse_from_indices(qn, kn, vn, ref_ids)) < TOL

    dense_attention(dq, dk, dv, out=out)
    assert _err(out, O.dense_causal(qn, kn, vn)) < TOL
    full = dense_attention(dq, dk, dv, causal=False)
    assert full.shape == q.shape and full.dtype == q.dtype
    ref_full = O.dense_causal(qn, kn, vn, causal=False)
    assert _err(full, ref_full) < TOL + 2.0 ** -8 * np.abs(ref_full).max()

    o1 = decode_dense(dq[:, :, -1:], dk, dv)
    assert o1.shape == (1, 3, 1, D)
    ref1 = O.dense_causal(qn[:, :, -1:], kn, vn, causal=False)
    assert _err(o1, ref1) < TOL + 2.0 ** -8 * np.abs(ref1).max()


def test_unbuilt_paths_refuse_other_head_dims(gpu_device):
    """vertical_and_slash (its estimator divides by the kernel's sqrt(D)) runs
    at 64, 96 and 128 only, the patched forward at the built head dims only;
    beyond 512 nothing runs."""
    from minference import streaming_forward
    from minference.ops.vertical_slash_kernel import vertical_and_slash_attention

    for d in (80, 256):
        q = torch.zeros(1, 2, 128, d, dtype=torch.bfloat16, device=gpu_device)
        with pytest.raises(NotImplementedError):
            vertical_and_slash_attention(q, q, q, 64, 64)
    q = torch.zeros(1, 2, 128, 600, dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(NotImplementedError):
        streaming_forward(q, q, q, 64, 128)


def test_head_dim_256_strided_and_fixed_ids(gpu_device):
    """D = 256: K read through the staged operands (a k view whose rows
    overlap is not read in place), S_q < S_k, bf16 outputs, and fixed block
    ids with repeats and ids out of range."""
    from minference import dense_attention, streaming_forward
    from minference.ops.block_sparse_kernel import block_sparse_attention_with_indices

    D, S_q, S_k = 256, 333, 900
    q, k, v = make_qkv(1, 2, S_q, S_k, D, torch.bfloat16, seed=256, sink_scale=8.0)
    dq, dk, dv = (t.to(gpu_device) for t in (q, k, v))
    qn, kn, vn = np32(q), np32(k), np32(v)
    out = torch.empty(q.shape, dtype=torch.float32, device=gpu_device)
    streaming_forward(dq, dk, dv, 32, 300, out=out)
    assert _err(out, O.streaming_attention(qn, kn, vn, 32, 300)) < TOL
    o16 = dense_attention(dq, dk, dv)
    ref = O.dense_causal(qn, kn, vn)
    assert o16.dtype == torch.bfloat16
    assert _err(o16, ref) < TOL + 2.0 ** -8 * np.abs(ref).max()
    n_bq, n_bk = -(-S_q // 64), -(-S_k // 64)
    ids = np.random.default_rng(5).integers(-2, n_bk + 2, size=(1, 2, n_bq, 6))
    block_sparse_attention_with_indices(dq, dk, dv, torch.from_numpy(ids), out=out)
    assert _err(out, O.block_sparse_from_indices(qn, kn, vn, ids)) < TOL
    # rows of k overlapping (row stride 128 < D): the kernels take staged K
    base = torch.randn(1, 2, S_k * 128 + 256, dtype=torch.bfloat16, device=gpu_device)
    ko = base.as_strided((1, 2, S_k, D), (2 * (S_k * 128 + 256), S_k * 128 + 256, 128, 1))
    streaming_forward(dq, ko, dv, 32, 300, out=out)
    kon = np32(ko.cpu())
    assert _err(out, O.streaming_attention(qn, kon, vn, 32, 300)) < TOL
