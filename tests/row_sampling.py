"""Row sampling for the full-length parity checks: one row in every query
block (or every few blocks) of every head, at an offset inside the block
that moves with the block and the head, checked against the oracle's
row-sampled fp64 attention (oracle.rows_attention) under the head's own
visibility rule."""

from __future__ import annotations

import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
from threadpoolctl import threadpool_limits

import oracle as O

DENSE, STREAM, BLOCK = 0, 1, 2  # MSA_KIND_DENSE, MSA_KIND_STREAM, MSA_KIND_BLOCK


def block_rows(S: int, h: int, every: int = 1, per_block: int = 1, extra=()) -> np.ndarray:
    """``per_block`` rows (evenly spaced, 64 of them = every row) of every
    ``every``-th query block bq, the first at offset (29 * bq + 7 * h + 3) mod
    64 so that the sampled offsets move with the block and the head; rows
    past S - 1 dropped; plus ``extra``."""
    bq = np.arange(0, -(-S // 64), every)
    base = (29 * bq + 7 * h + 3) % 64
    off = (base[:, None] + (64 // per_block) * np.arange(per_block)[None, :]) % 64
    r = (bq[:, None] * 64 + off).ravel()
    ex = np.array([x for x in extra if 0 <= x < S], dtype=np.int64)
    return np.unique(np.concatenate([r[r < S].astype(np.int64), ex]))


def head_rows_reference(qh, kh, vh, rows, kind, p1, p2, scale, ids=None, cnt=None):
    """fp64 oracle output of ``rows`` of one head of the given kind
    (stream_llm p1 = n_init, p2 = n_local; block_sparse from ids / cnt)."""
    if kind == STREAM:
        vis, keys = O.stream_rows_visible(p1, p2)
    elif kind == BLOCK:
        vis, keys = O.block_rows_visible(ids, cnt, qh.shape[0])
    elif kind == DENSE:
        vis, keys = O.causal_rows_visible, None
    else:
        raise ValueError(f"no row rule for head kind {kind}")
    return O.rows_attention(qh, kh, vh, rows, vis, scale, keys=keys)


def map_heads(fn, heads, workers: int = 8, tag: str = ""):
    """fn(h) for every head on a thread pool (numpy's products and
    element-wise passes release the GIL), two BLAS threads per worker (16
    threads: the GPU box's CPU share); returns the results in order and
    prints the elapsed time."""
    t0 = time.time()
    with threadpool_limits(2), ThreadPoolExecutor(max_workers=workers) as ex:
        res = list(ex.map(fn, heads))
    print(f"{tag} {len(res)} heads checked in {time.time() - t0:.1f} s", flush=True)
    return res
