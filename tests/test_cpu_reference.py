"""The torch-CPU restatement of the reference's CPU paths (timed as the
benchmark's CPU baseline) against the numpy oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from msa_data import make_qkv, np32
from oracle import cpu_reference as R


@pytest.mark.parametrize("S,n_init,n_local,D", [(1000, 64, 256, 96), (700, 0, 128, 64),
                                                (300, 400, 64, 96)])
def test_streaming_reference_matches_oracle(S, n_init, n_local, D):
    q, k, v = make_qkv(1, 3, S, S, D, torch.float32, seed=S)
    got = R.streaming_reference(q, k, v, n_init, n_local).numpy()
    ref = O.streaming_attention(np32(q), np32(k), np32(v), n_init, n_local)
    assert np.abs(got - ref).max() < 1e-5


@pytest.mark.parametrize("S,topk,D,block", [(1000, 4, 96, 64), (640, 100, 64, 64),
                                             (1000, 3, 96, 128), (1100, 2, 96, 256),
                                             (1500, 2, 64, 512), (1000, 3, 96, 192),
                                             (1600, 2, 96, 320)])
def test_block_reference_matches_oracle(S, topk, D, block):
    q, k, v = make_qkv(1, 2, S, S, D, torch.bfloat16, seed=7, sink_scale=8.0)
    ids = R.select_blocks(R._padded(q), R._padded(k), topk, block).numpy()
    ridx, rcnt = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, "bf16", block=block)
    assert np.array_equal(rcnt[0], O.attend_count(ridx, S, S, block)[0])
    for h in range(2):
        for bq in range(ridx.shape[2]):
            c = rcnt[0, h, bq]
            assert set(ridx[0, h, bq, :c]) == set(x for x in ids[0, h, bq] if x <= bq)
    got = R.block_sparse_reference(q.float(), k.float(), v.float(), topk, block).numpy()
    # the fp32 inputs pool in fp32: select on the same values for the oracle
    ridx32, _ = O.select_block_sparse_topk_indices(np32(q), np32(k), topk, "fp32", block=block)
    ref = O.block_sparse_from_indices(np32(q), np32(k), np32(v), ridx32, block=block)
    assert np.abs(got - ref).max() < 1e-5
