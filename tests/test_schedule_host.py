"""Host logic of the layer schedule (launch_block_layer) on the CPU: the
library calls and the streams they go to, recorded by test doubles of the
C ABI wrapper and of torch's stream API (no GPU).  The GPU tests check that
the schedule computes what the plain calls compute."""

from __future__ import annotations

import contextlib

import torch

from minference import _abi
from minference.modules import minference_forward as mf


class _Stream:
    def __init__(self, name, log):
        self.name, self.log = name, log

    def wait_stream(self, other):
        self.log.append(("wait", self.name, other.name))


def test_block_layer_schedule(monkeypatch):
    log = []
    main = _Stream("main", log)
    current = [main]

    @contextlib.contextmanager
    def stream_ctx(st):
        current.append(st)
        try:
            yield
        finally:
            current.pop()

    monkeypatch.setattr(mf, "_SIDE_STREAMS", {})
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device=None: main)
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(torch.cuda, "Stream", lambda device=None: _Stream("side", log))
    monkeypatch.setattr(torch.cuda, "stream", stream_ctx)

    def block_estimate(q, k, heads, topk, topk_max, scale, idx, cnt, ws=None, flags=0):
        log.append(("estimate", current[-1].name, flags, tuple(heads), ws is not None))

    def stage_kv(k, v, ws, kv_heads=None):
        log.append(("stage", current[-1].name))

    def stage_kv_pool(q, k, v, slot_heads, est_ws, ws):
        log.append(("stage+pool", current[-1].name, tuple(slot_heads), est_ws))

    def layer_attention(q, k, v, out, heads, **kw):
        log.append(("attention", current[-1].name, len(heads), kw.get("staged"),
                    kw.get("idx_slots")))

    monkeypatch.setattr(mf._abi, "block_estimate", block_estimate)
    monkeypatch.setattr(mf._abi, "stage_kv", stage_kv)
    monkeypatch.setattr(mf._abi, "stage_kv_pool", stage_kv_pool)
    monkeypatch.setattr(mf._abi, "layer_attention", layer_attention)

    pats = {0: ["stream_llm", 64, 256, 1], 1: ["block_sparse", 4, 0, 1], 2: ["dense", 0, 0, 1],
            3: ["block_sparse", 2, 0, 1]}
    plan = mf.build_layer_plan(pats, 4, 96, 1024)
    q = torch.zeros(1, 4, 1024, 96)
    marks = []
    mf.launch_block_layer(q, q, q, plan, q, None, None, None, "est-ws",
                          flags=_abi.MSA_SELECT_FORCE_DIAG,
                          mark=lambda name, st: marks.append((name, st.name)))
    select = _abi.MSA_ESTIMATE_SELECT_ONLY | _abi.MSA_SELECT_FORCE_DIAG
    assert log == [
        ("stage+pool", "main", (1, 3), "est-ws"),       # staging + pooling, one launch
        ("estimate", "main", select, (1, 3), True),     # then the selection, same stream
        ("attention", "main", 4, True, 2),              # one launch of all heads
    ]
    # one stream, no cross-stream waits
    assert [m[0] for m in marks] == ["start", "stage0", "stage1", "est0", "est1", "attn0",
                                     "attn0_end"]
    assert {st for _, st in marks} == {"main"}


def test_tile_ids_keep_token_visibility():
    """Ids of 128- to 512-token blocks expanded to 64-token tiles select the
    same (query, key) pairs: chunked and ragged shapes, ids out of range,
    negative and repeated."""
    import numpy as np

    import oracle as O
    from minference.ops.block_sparse_kernel import canonical_block_lists, tile_ids

    g = np.random.default_rng(3)
    for block, s_q, s_k in [(128, 300, 300), (256, 1000, 1000), (512, 700, 1500),
                            (128, 100, 900), (256, 64, 64), (192, 500, 500), (320, 300, 1000)]:
        n_bq, n_bk = -(-s_q // block), -(-s_k // block)
        ids = g.integers(-2, n_bk + 2, size=(1, 2, n_bq, 4))
        n_qt, n_kt = -(-s_q // 64), -(-s_k // 64)
        tiles = tile_ids(torch.from_numpy(ids), block, n_qt)
        assert tiles.shape == (1, 2, n_qt, 4 * block // 64)
        lists, cnt = canonical_block_lists(tiles, n_kt)
        for h in range(2):
            want = O.block_token_visible(ids[0, h], s_q, s_k, block)
            got = O.block_token_visible(tiles[0, h].numpy(), s_q, s_k, 64)
            assert np.array_equal(got, want)
            # the canonical lists: the distinct in-range tiles, ascending
            for t in range(n_qt):
                c = int(cnt[0, h, t])
                row = tiles[0, h, t].numpy()
                assert lists[0, h, t, :c].tolist() == sorted(set(row[(row >= 0) & (row < n_kt)]))
