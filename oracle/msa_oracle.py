"""numpy restatement of the reference's sparse prefill attention semantics.

TEST INFRASTRUCTURE ONLY: the checker, never the thing measured or shipped.

Reference files (paths relative to /root/reference/MInference-NPU/):
  streaming  : minference/ops/streaming_kernel_npu.py:94-146 (CPU path), :349-397 (entry)
  block      : minference/ops/block_sparse_kernel_npu.py:230-263 (selector),
               :266-317 (token mask), :325-348 (CPU path), :609-709 (entry)
  dense      : minference/backend_npu/attention.py:166-189 (CPU path), :192-255 (entry)
  dispatch   : minference/modules/minference_forward.py:384-487

Parity pins (each function is checked by tests/test_oracle.py against
something other than its own formula):
  pool_blocks         : torch's bf16/fp16 ``mean(dim=3)`` (the library call the
                        reference makes), bit for bit
  block_scores /
  select_topk         : brute-force pure-Python loops; sortedness and causal
                        count invariants (tests/test_block_sparse_kernel.py:186-211
                        in the reference); constructed known answers (monotone
                        scores, exact ties); torch.topk on torch.matmul scores
                        with a near-tie exemption
  streaming_attention : per-row brute force (reference tests/test_streaming_kernel.py:79-117);
                        Q = 0 closed form (uniform mean over the visible set);
                        n_local >= S equals causal dense; LSE-merge identity
  block_sparse_from_indices : full top-k equals causal dense; Q = 0 closed form;
                        per-row brute force over the expanded token set
  dense_causal        : torch scaled_dot_product_attention in fp64 (is_causal
                        True and False)
  rows_attention and the *_rows_visible rules : every row of small heads equal to
                        streaming_attention / block_sparse_from_indices /
                        dense_causal, rows given in any grouping
  rope_rotate_half    : HF Phi-3's apply_rotary_pos_emb on CPU torch in bf16 / fp16
                        (the call the reference makes), bit for bit, full and
                        partial rotary; in fp64 a norm-preserving rotation of
                        the (i, i + rot/2) pairs
"""

from __future__ import annotations

import math
from typing import Sequence

import numpy as np

__all__ = [
    "ALLOWED_HEAD_DIMS",
    "next_allowed_head_dim",
    "sparse_scale",
    "dense_scale",
    "bf16_round",
    "f16_round",
    "round_to",
    "pool_blocks",
    "block_scores",
    "select_topk",
    "select_block_sparse_topk_indices",
    "attend_count",
    "vs_sizes",
    "vs_logits",
    "vs_probs",
    "vs_diagonal_sums",
    "vs_scores",
    "vs_estimate",
    "vs_token_visible",
    "vs_row_visible",
    "vertical_slash_from_indices",
    "stream_visible",
    "streaming_attention",
    "block_token_visible",
    "block_sparse_from_indices",
    "dense_causal",
    "masked_attention",
    "rows_attention",
    "stream_rows_visible",
    "block_rows_visible",
    "causal_rows_visible",
    "layer_attention",
    "stream_pairs",
    "block_tiles",
    "causal_pairs",
    "rope_rotate_half",
]

BLOCK = 64
ALLOWED_HEAD_DIMS = (16, 32, 64, 128, 256, 512)


# ---------------------------------------------------------------------------
# scale quirk
# ---------------------------------------------------------------------------
def next_allowed_head_dim(d: int) -> int:
    """Head dims are zero-padded to the next of (16, 32, 64, 128, 256, 512)
    before the sparse ops compute their scale
    (streaming_kernel_npu.py:70-86, 377-381; block_sparse_kernel_npu.py:95-101, 651-656)."""
    for cand in ALLOWED_HEAD_DIMS:
        if cand >= d:
            return cand
    raise ValueError(f"head_dim={d} exceeds {ALLOWED_HEAD_DIMS[-1]}")


def sparse_scale(d: int) -> float:
    """Softmax (and selector score) scale of stream_llm / block_sparse heads:
    Dp ** -0.5 with Dp the padded dim (streaming_kernel_npu.py:114;
    block_sparse_kernel_npu.py:254, 340).  Zero padding leaves q.k unchanged,
    so only the scale differs from the unpadded computation."""
    return next_allowed_head_dim(d) ** -0.5


def dense_scale(d: int) -> float:
    """dense_attention's default scale 1/sqrt(D) on unpadded D (attention.py:210-211)."""
    return 1.0 / math.sqrt(d)


# ---------------------------------------------------------------------------
# rounding
# ---------------------------------------------------------------------------
def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 round-to-nearest-even, returned as float32 values."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nonfinite = (u & 0x7F800000) == 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    r = np.where(nonfinite, u & 0xFFFF0000, r).astype(np.uint32)
    return r.view(np.float32)


def f16_round(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_round(x)
    if dtype == "fp16":
        return f16_round(x)
    if dtype == "fp32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# rotary embedding (minference_forward.py:205-212 looks up the model module's
# apply_rotary_pos_emb, :336-341 calls it; HF Phi-3 / Llama rotate-half form)
# ---------------------------------------------------------------------------
def rope_rotate_half(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """x * cos + rotate_half(x) * sin on the first rot = cos.shape[-1] dims,
    the rest passed through, with the eager op-by-op rounding of 16-bit
    tensors: each product and the sum are computed in fp32 and rounded to
    ``dtype``.  x [B, H, S, D]; cos, sin [B or 1, S, rot]; all float32
    holding ``dtype`` values."""
    x = np.asarray(x, dtype=np.float32)
    c = np.asarray(cos, dtype=np.float32)[:, None]
    s = np.asarray(sin, dtype=np.float32)[:, None]
    rot = c.shape[-1]
    half = rot // 2
    x1, x2 = x[..., :half], x[..., half:rot]
    r = lambda a: round_to(a, dtype)  # noqa: E731
    out = x.copy()
    out[..., :half] = r(r(x1 * c[..., :half]) - r(x2 * s[..., :half]))
    out[..., half:rot] = r(r(x2 * c[..., half:]) + r(x1 * s[..., half:]))
    return out


# ---------------------------------------------------------------------------
# block selector (block_sparse_kernel_npu.py:230-263)
# ---------------------------------------------------------------------------
def pool_blocks(x: np.ndarray, dtype: str, block: int = BLOCK) -> np.ndarray:
    """Mean over consecutive ``block`` rows of x [..., S, D] in the input dtype.

    The last partial block is zero padded and still divided by ``block``
    (F.pad then reshape().mean(dim=3), :240-251).  The sum is formed in fp64
    (exact for 16-bit inputs), rounded to fp32, divided by ``block`` and
    rounded to the input dtype, which is what torch's CPU bf16/fp16 mean
    produces; the result is returned as float32 (the ``.to(fp32)`` at :251).
    """
    x = np.asarray(x, dtype=np.float32)
    S = x.shape[-2]
    pad = (-S) % block
    if pad:
        widths = [(0, 0)] * (x.ndim - 2) + [(0, pad), (0, 0)]
        x = np.pad(x, widths)
    nb = x.shape[-2] // block
    xr = x.reshape(*x.shape[:-2], nb, block, x.shape[-1]).astype(np.float64)
    s = xr.sum(axis=-2).astype(np.float32)
    mean = (s / np.float32(block)).astype(np.float32)
    return round_to(mean, dtype)


def block_scores(q_pool: np.ndarray, k_pool: np.ndarray, scale: float) -> np.ndarray:
    """fp32 pooled scores q_pool . k_pool^T * scale with the block-causal mask
    (bk > bq -> -inf, q-block frame) of :253-260.  The dot product is formed
    in fp64 and rounded once to fp32 (exact for 16-bit pooled operands)."""
    s = np.matmul(q_pool.astype(np.float64), np.swapaxes(k_pool.astype(np.float64), -1, -2))
    s = s.astype(np.float32) * np.float32(scale)
    n_bq, n_bk = s.shape[-2], s.shape[-1]
    causal = np.arange(n_bq)[:, None] >= np.arange(n_bk)[None, :]
    return np.where(causal, s, np.float32(-np.inf)).astype(np.float32)


def select_topk(scores: np.ndarray, topk: int, force_first: bool = False,
                force_diag: bool = False):
    """Per query block: the ``topk`` largest scores, ties -> lower block id.

    Returns (idx, cnt).  idx[..., bq, :cnt] are the selected causal ids
    ascending (what torch.topk(...).indices.sort() yields on the causal part);
    cnt = min(topk, bq + 1).  The reference fills the remaining slots with
    -inf future ids chosen by torch.topk internals (:262-263); they are never
    attended (token causal mask, :281-284), and here they are the next
    future ids bq+1, bq+2, ... in ascending order.

    NaN scores rank above +inf, all NaNs alike, ties to the lower id
    (torch.topk, which the reference calls at :262, returns NaN entries
    first: topk([1, nan, 2, inf, nan], 3) gives ids 1, 4, 3).

    force_first / force_diag (this build's selector option, not the
    reference's): block 0 / block bq rank above every scored block,
    NaN included, inside the top-k; between them the lower id wins.
    """
    *lead, n_bq, n_bk = scores.shape
    # rank classes: 2 = forced, 1 = NaN, 0 = scored (ordered by value)
    cls = np.where(np.isnan(scores), 1, 0).astype(np.int8)
    if force_first or force_diag:
        if force_first:
            cls[..., :, 0] = 2
        if force_diag:
            d = np.arange(min(n_bq, n_bk))
            cls[..., d, d] = 2
    topk = min(int(topk), n_bk)
    flat = scores.reshape(-1, n_bq, n_bk)
    fcls = cls.reshape(-1, n_bq, n_bk)
    idx = np.empty((flat.shape[0], n_bq, topk), dtype=np.int64)
    cnt = np.empty((flat.shape[0], n_bq), dtype=np.int64)
    for bq in range(n_bq):
        n = min(bq + 1, n_bk)
        c = min(topk, n)
        row = flat[:, bq, :n].astype(np.float64)
        rcls = fcls[:, bq, :n]
        val = np.where(rcls == 0, row, 0.0) + 0.0  # -0 ranks with +0
        ids = np.broadcast_to(np.arange(n), row.shape)
        # class descending, then value descending, then id ascending
        order = np.lexsort((ids, -val, -rcls), axis=-1)[:, :c]
        sel = np.sort(order, axis=-1)
        idx[:, bq, :c] = sel
        if c < topk:
            idx[:, bq, c:] = bq + 1 + np.arange(topk - c)
        cnt[:, bq] = c
    return idx.reshape(*lead, n_bq, topk), cnt.reshape(*lead, n_bq)


def select_block_sparse_topk_indices(q: np.ndarray, k: np.ndarray, topk_blocks: int,
                                     dtype: str, scale: float | None = None,
                                     block: int = BLOCK, force_first: bool = False,
                                     force_diag: bool = False):
    """Full selector on [..., S, D] inputs (block_sparse_kernel_npu.py:230-263)."""
    if scale is None:
        scale = sparse_scale(q.shape[-1])
    qp = pool_blocks(q, dtype, block)
    kp = pool_blocks(k, dtype, block)
    return select_topk(block_scores(qp, kp, scale), max(1, int(topk_blocks)),
                       force_first, force_diag)


def attend_count(idx: np.ndarray, s_q: int, s_k: int, block: int = BLOCK) -> np.ndarray:
    """Per id row [..., n_bq, topk] (ascending): how many ids some row of the
    query block can attend under the absolute token-causal mask, row i at
    s_k - s_q + i (block_sparse_kernel_npu.py:310-314).  An id counts when
    its first key is at or before the block's last row; the counted ids are a
    prefix of the row.  With s_q == s_k this is min(topk, bq + 1); with
    s_q < s_k it includes surplus (q-frame future) ids in the rows' past."""
    idx = np.asarray(idx)
    n_bq = idx.shape[-2]
    last = s_k - s_q + np.minimum(np.arange(n_bq) * block + block - 1, s_q - 1)
    return (idx * block <= last[:, None]).sum(-1)


# ---------------------------------------------------------------------------
# vertical_and_slash estimator (minference_forward.py:140-167)
# ---------------------------------------------------------------------------
LAST_Q = 64          # query rows the estimator looks at (minference_forward.py:43)
VS_SINK_COLS = 30    # columns forced into the vertical set (:157)
VS_LOCAL_DIAGS = 100  # nearest diagonals forced into the slash set (:163)


def vs_sizes(s: int, vertical_size: int, slash_size: int):
    """Clamped sizes of :146-147: min(S, max(v, 30)) and min(S, max(s, 50))."""
    return min(s, max(int(vertical_size), 30)), min(s, max(int(slash_size), 50))


def vs_logits(q: np.ndarray, k: np.ndarray, dtype: str) -> np.ndarray:
    """Last-rows logits of one head (:149-151), q, k [S, D] with S_q == S_k:
    q[-n:] . k^T formed in fp64 (exact for 16-bit operands), rounded to fp32
    and to the input dtype (the reference's matmul output dtype), divided by
    fp32(sqrt(D)) and rounded to the input dtype again (``/ math.sqrt(D)`` on
    a bf16/fp16 tensor); the last n columns carry the causal mask (row r
    sees column S - n + c iff c <= r) as -inf.  Returns x [n, S] fp64."""
    S, D = k.shape
    n = min(LAST_Q, S)
    ql = np.asarray(q[S - n:], dtype=np.float64)
    dots = ql @ np.asarray(k, dtype=np.float64).T                    # [n, S]
    a = round_to(dots.astype(np.float32), dtype)
    x = round_to(a / np.float32(math.sqrt(D)), dtype).astype(np.float64)
    r = np.arange(n)[:, None]
    c = np.arange(S)[None, :] - (S - n)
    return np.where(c > r, -np.inf, x)


def vs_probs(x: np.ndarray) -> np.ndarray:
    """Row softmax of vs_logits in fp64 (the reference's fp32 softmax of
    :152, here without its rounding)."""
    m = x.max(axis=1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=1, keepdims=True)


def vs_diagonal_sums(p: np.ndarray) -> np.ndarray:
    """Sums of p [n, S] along each diagonal t = 0 .. S-1 in fp64: element
    (i, i + t + 1 - n) for every row i where that column exists
    (sum_all_diagonal_matrix's output, :124-137, truncated at :161-162)."""
    n, S = p.shape
    slash = np.zeros(S)
    for i in range(n):
        lo = n - 1 - i                     # first diagonal that meets row i
        slash[lo:] += p[i, : S - lo]
    return slash


def vs_scores(q: np.ndarray, k: np.ndarray, dtype: str):
    """Column sums and anti-diagonal sums of the last-rows attention of one
    head (:148-164).  q, k: [S, D] with S_q == S_k.

    * the logits of vs_logits;
    * softmax in fp64 (vs_probs), then column sums and the diagonal sums of
      vs_diagonal_sums, each rounded once to fp32;
    * the first 30 columns and the last 100 diagonals are set to +inf.

    Returns (vertical [S] fp32, slash [S] fp32)."""
    S = k.shape[0]
    p = vs_probs(vs_logits(q, k, dtype))
    vert = p.sum(axis=0).astype(np.float32)
    slash = vs_diagonal_sums(p).astype(np.float32)
    vert[:VS_SINK_COLS] = np.inf
    slash[max(0, S - VS_LOCAL_DIAGS):] = np.inf
    return vert, slash


def _topk_lower(vals: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest values, ties to the lower index."""
    return np.argsort(-vals.astype(np.float64), kind="stable")[:k]


def vs_estimate(q: np.ndarray, k: np.ndarray, vertical_size: int, slash_size: int,
                dtype: str):
    """Vertical and slash indices of every head (:140-165).  q [B, H, S, D],
    k [B, H_kv, S, D].  Returns (v_idx [B, H, nv] ascending, s_idx [B, H, ns]
    descending), nv/ns from vs_sizes; s = S - 1 - t for the selected
    diagonals t.  Ties in the top-k go to the lower column / diagonal index
    (torch.topk's choice among exact ties is unspecified)."""
    B, H, S, D = q.shape
    assert k.shape[2] == S, "vertical_and_slash needs S_q == S_k"
    kvg = H // k.shape[1]
    nv, ns = vs_sizes(S, vertical_size, slash_size)
    v_idx = np.empty((B, H, nv), dtype=np.int64)
    s_idx = np.empty((B, H, ns), dtype=np.int64)
    for b, h in _heads(q):
        vert, slash = vs_scores(q[b, h], k[b, h // kvg], dtype)
        v_idx[b, h] = np.sort(_topk_lower(vert, nv))
        s_idx[b, h] = np.sort(S - 1 - _topk_lower(slash, ns))[::-1]
    return v_idx, s_idx


# ---------------------------------------------------------------------------
# token visibility
# ---------------------------------------------------------------------------
def stream_visible(s_q: int, s_k: int, n_init: int, n_local: int) -> np.ndarray:
    """visible(i, j) = j <= a and (j > a - n_local or j < n_init),
    a = S_k - S_q + i (streaming_kernel_npu.py:127-136)."""
    a = np.arange(s_k - s_q, s_k)[:, None]
    j = np.arange(s_k)[None, :]
    return (j <= a) & ((j > a - n_local) | (j < n_init))


def block_token_visible(idx_row: np.ndarray, s_q: int, s_k: int, block: int = BLOCK) -> np.ndarray:
    """Token mask of one head from block ids idx_row [n_bq, topk]
    (block_sparse_kernel_npu.py:266-317; True = visible)."""
    n_bq = idx_row.shape[0]
    n_bk = -(-s_k // block)
    attend = np.zeros((n_bq, n_bk), dtype=bool)
    for bq in range(n_bq):
        ids = idx_row[bq]
        ids = ids[(ids >= 0) & (ids < n_bk)]
        attend[bq, ids] = True
    tok = np.repeat(np.repeat(attend, block, axis=0), block, axis=1)[:s_q, :s_k]
    a = np.arange(s_k - s_q, s_k)[:, None]
    j = np.arange(s_k)[None, :]
    return tok & (j <= a)


def vs_token_visible(v_idx_row: np.ndarray, s_idx_row: np.ndarray, s_q: int, s_k: int,
                     block: int = BLOCK) -> np.ndarray:
    """Token mask of one vertical_and_slash head (vertical_slash_kernel_npu.py:
    282-367, the reference's production path; True = visible).  Query block
    bq (end_m = 64(bq+1)) sees, for every slash s < end_m, the 64 keys
    [hi - 64, hi) with hi = clamp(end_m - s, 64, S_k); every row sees the
    vertical columns (clamped into [0, S_k)); then the causal mask j <= i."""
    assert s_q == s_k, "vertical_and_slash needs S_q == S_k"
    n_rows = -(-s_k // block)
    cov = np.zeros((n_rows, s_k), dtype=bool)
    for bq in range(n_rows):
        end_m = (bq + 1) * block
        for s in np.asarray(s_idx_row).tolist():
            if s < end_m:
                hi = min(max(end_m - s, block), s_k)
                lo = min(max(hi - block, 0), s_k)
                cov[bq, lo:hi] = True
    vert = np.zeros(s_k, dtype=bool)
    vert[np.clip(np.asarray(v_idx_row), 0, s_k - 1)] = True
    tok = np.repeat(cov | vert[None, :], block, axis=0)[:s_q]
    i = np.arange(s_q)[:, None]
    j = np.arange(s_k)[None, :]
    return tok & (j <= i)


def vs_row_visible(v_idx_row: np.ndarray, s_idx_row: np.ndarray, row: int, s_k: int,
                   block: int = BLOCK) -> np.ndarray:
    """Key ids (ascending) that query row ``row`` of a vertical_and_slash head
    sees: row ``row`` of vs_token_visible without building the S x S mask
    (same rule: the slash windows of its 64-row block, the vertical columns,
    then j <= row)."""
    end_m = (row // block + 1) * block
    keys = [np.clip(np.asarray(v_idx_row, dtype=np.int64), 0, s_k - 1)]
    s = np.asarray(s_idx_row, dtype=np.int64)
    s = s[s < end_m]
    hi = np.minimum(np.maximum(end_m - s, block), s_k)
    lo = np.minimum(np.maximum(hi - block, 0), s_k)
    for a, b in zip(lo.tolist(), hi.tolist()):
        keys.append(np.arange(a, b))
    js = np.unique(np.concatenate(keys))
    return js[js <= row]


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------
def masked_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, visible: np.ndarray,
                     scale: float, acc=np.float64) -> np.ndarray:
    """softmax(q k^T * scale, masked) v with fully masked rows -> 0
    (the reference's nan_to_num, streaming_kernel_npu.py:142,
    block_sparse_kernel_npu.py:346).  q [S_q, D], k/v [S_k, D]."""
    logits = (q.astype(acc) @ k.astype(acc).T) * acc(scale)
    logits = np.where(visible, logits, -np.inf)
    m = logits.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(logits - m)
    den = p.sum(axis=-1, keepdims=True)
    out = (p @ v.astype(acc)) / np.where(den > 0, den, 1.0)
    return np.where(den > 0, out, 0.0).astype(acc)


def rows_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, rows: np.ndarray, visible,
                   scale: float, keys=None, group: int = 64, acc=np.float64) -> np.ndarray:
    """Output rows ``rows`` of one head (q [S_q, D], k/v [S_k, D], S_q == S_k):
    masked_attention restricted to those rows, ``group`` rows at a time, for
    full-length checks that sample rows.  ``visible(rows_g, keys_g) -> bool
    [len(rows_g), len(keys_g)]`` is the head's token visibility;
    ``keys(rows_g)`` (ascending key ids that may be visible to any of the
    rows; default every key up to the last row) only narrows the product.
    Rows that see no key give 0 (masked_attention's rule).  The logits and
    the gathered keys / values live in buffers reused across groups."""
    rows = np.asarray(rows, dtype=np.int64)
    D = q.shape[1]
    out = np.zeros((rows.size, D), dtype=acc)
    bufs = {}

    def buf(name, shape, dtype):
        n = int(np.prod(shape))
        b = bufs.get(name)
        if b is None or b.size < n:
            b = bufs[name] = np.empty(max(n, 2 * (0 if b is None else b.size)), dtype=dtype)
        return b[:n].reshape(shape)

    for g0 in range(0, rows.size, group):
        rg = rows[g0:g0 + group]
        kg = np.arange(int(rg.max()) + 1) if keys is None else np.asarray(keys(rg), np.int64)
        n = kg.size
        if n == 0:
            continue
        kk, vv = buf("k", (n, D), acc), buf("v", (n, D), acc)
        if kg[-1] - kg[0] + 1 == n:            # a key range
            kk[...] = k[kg[0]:kg[-1] + 1]
            vv[...] = v[kg[0]:kg[-1] + 1]
        else:
            kk[...] = np.take(k, kg, axis=0, out=buf("g", (n, D), k.dtype))
            vv[...] = np.take(v, kg, axis=0, out=buf("g", (n, D), v.dtype))
        lg = buf("lg", (rg.size, n), acc)
        np.matmul(q[rg].astype(acc), kk.T, out=lg)
        lg *= acc(scale)
        np.copyto(lg, -np.inf, where=np.logical_not(visible(rg, kg)))
        m = lg.max(axis=-1)
        m = np.where(np.isfinite(m), m, 0.0)
        lg -= m[:, None]
        np.exp(lg, out=lg)
        den = lg.sum(axis=-1)
        o = lg @ vv
        out[g0:g0 + rg.size] = np.where(den[:, None] > 0, o / np.where(den > 0, den, 1.0)[:, None],
                                        0.0)
    return out


def stream_rows_visible(n_init: int, n_local: int):
    """visible(rows, keys) and keys(rows) of a stream_llm head (S_q == S_k):
    j <= i and (j > i - n_local or j < n_init), stream_visible's rule."""
    def visible(rows, keys):
        a = rows[:, None]
        j = keys[None, :]
        return (j <= a) & ((j > a - n_local) | (j < n_init))

    def keys(rows):
        lo = max(0, int(rows.min()) - n_local + 1)
        return np.concatenate([np.arange(min(n_init, lo)), np.arange(lo, int(rows.max()) + 1)])

    return visible, keys


def block_rows_visible(idx_row: np.ndarray, cnt_row: np.ndarray | None, s_k: int,
                       block: int = BLOCK):
    """visible(rows, keys) and keys(rows) of a block_sparse head from its ids
    idx_row [n_bq, topk] (the first cnt_row[bq] of each row when given; ids
    outside [0, n_kv_blocks) ignored) intersected with j <= i:
    block_token_visible's rule (S_q == S_k).  keys(rows) lists the keys of
    the blocks any of the rows attends."""
    n_bq = idx_row.shape[0]
    n_bk = -(-s_k // block)
    ids = np.asarray(idx_row, dtype=np.int64)
    use = (ids >= 0) & (ids < n_bk)
    if cnt_row is not None:
        use &= np.arange(ids.shape[1])[None, :] < np.asarray(cnt_row)[:, None]
    attend = np.zeros((n_bq, n_bk), dtype=bool)
    r, c = np.nonzero(use)
    attend[r, ids[r, c]] = True

    def visible(rows, keys):
        return attend[(rows // block)[:, None], (keys // block)[None, :]] & (keys[None, :] <= rows[:, None])

    def keys(rows):
        blocks = np.nonzero(attend[rows // block].any(axis=0))[0]
        js = (blocks[:, None] * block + np.arange(block)[None, :]).ravel()
        return js[js <= int(rows.max())]

    return visible, keys


def causal_rows_visible(rows, keys):
    """visible(rows, keys) of a causal dense head: j <= i."""
    return keys[None, :] <= rows[:, None]


def _heads(x: np.ndarray):
    """[B, H, S, D] -> iterator of (b, h)."""
    B, H = x.shape[0], x.shape[1]
    for b in range(B):
        for h in range(H):
            yield b, h


def streaming_attention(q, k, v, n_init: int, n_local: int, scale: float | None = None,
                        acc=np.float64, chunk_size_q: int | None = None) -> np.ndarray:
    """stream_llm output for [B, H, S, D] inputs (streaming_kernel_npu.py:94-146),
    chunked over queries with the reference's rule
    chunk = max(64, min(S_q, 4M // S_k)) (:116-117)."""
    if scale is None:
        scale = sparse_scale(q.shape[-1])
    B, H, s_q, D = q.shape
    s_k = k.shape[2]
    kvg = H // k.shape[1]
    if chunk_size_q is None:
        chunk_size_q = max(64, min(s_q, (4 * 1024 * 1024) // max(1, s_k)))
    out = np.zeros((B, H, s_q, D), dtype=acc)
    for b, h in _heads(q):
        for c0 in range(0, s_q, chunk_size_q):
            c1 = min(c0 + chunk_size_q, s_q)
            a = np.arange(s_k - s_q + c0, s_k - s_q + c1)[:, None]
            j = np.arange(s_k)[None, :]
            vis = (j <= a) & ((j > a - n_local) | (j < n_init))
            out[b, h, c0:c1] = masked_attention(q[b, h, c0:c1], k[b, h // kvg], v[b, h // kvg],
                                                vis, scale, acc)
    return out


def block_sparse_from_indices(q, k, v, idx, scale: float | None = None,
                              acc=np.float64, block: int = BLOCK) -> np.ndarray:
    """Block-sparse attention for fixed ids idx [B, H, n_bq, topk] of
    ``block``-token blocks (reference tests/test_block_sparse_kernel.py:96-119
    semantics; the ids are expanded to tokens and intersected with the token
    causal mask)."""
    if scale is None:
        scale = sparse_scale(q.shape[-1])
    B, H, s_q, D = q.shape
    s_k = k.shape[2]
    kvg = H // k.shape[1]
    out = np.zeros((B, H, s_q, D), dtype=acc)
    for b, h in _heads(q):
        vis = block_token_visible(np.asarray(idx[b, h]), s_q, s_k, block)
        out[b, h] = masked_attention(q[b, h], k[b, h // kvg], v[b, h // kvg], vis, scale, acc)
    return out


def vertical_slash_from_indices(q, k, v, v_idx, s_idx, scale: float | None = None,
                                acc=np.float64) -> np.ndarray:
    """Vertical-slash attention for given indices v_idx [B, H, nv] and s_idx
    [B, H, ns] (_vertical_slash_pytorch_ref, vertical_slash_kernel_npu.py:375-407;
    scale (padded D)**-0.5 after the pad at :581-587)."""
    if scale is None:
        scale = sparse_scale(q.shape[-1])
    B, H, s_q, D = q.shape
    s_k = k.shape[2]
    kvg = H // k.shape[1]
    out = np.zeros((B, H, s_q, D), dtype=acc)
    for b, h in _heads(q):
        vis = vs_token_visible(v_idx[b, h], s_idx[b, h], s_q, s_k)
        out[b, h] = masked_attention(q[b, h], k[b, h // kvg], v[b, h // kvg], vis, scale, acc)
    return out


def dense_causal(q, k, v, scale: float | None = None, acc=np.float64,
                 causal: bool = True) -> np.ndarray:
    """Dense attention (attention.py:166-189): causal j <= i + (S_k - S_q), or
    with causal=False every key for every query (any S_q, S_k)."""
    if scale is None:
        scale = dense_scale(q.shape[-1])
    B, H, s_q, D = q.shape
    s_k = k.shape[2]
    kvg = H // k.shape[1]
    a = np.arange(s_k - s_q, s_k)[:, None]
    vis = np.arange(s_k)[None, :] <= a
    if not causal:
        vis = np.ones((s_q, s_k), dtype=bool)
    out = np.zeros((B, H, s_q, D), dtype=acc)
    for b, h in _heads(q):
        out[b, h] = masked_attention(q[b, h], k[b, h // kvg], v[b, h // kvg], vis, scale, acc)
    return out


def layer_attention(q, k, v, patterns: Sequence[tuple], dtype: str,
                    acc=np.float64):
    """One patched layer (minference_forward.py:398-487): per head h,
    patterns[h] = (type, p1, p2).  Returns (out, {head: (idx, cnt)})."""
    B, H, s_q, D = q.shape
    kvg = H // k.shape[1]
    out = np.zeros((B, H, s_q, D), dtype=acc)
    sel = {}
    for h in range(H):
        ty, p1, p2 = patterns[h][:3]
        qh, kh, vh = q[:, h:h + 1], k[:, h // kvg:h // kvg + 1], v[:, h // kvg:h // kvg + 1]
        if ty == "stream_llm":
            out[:, h:h + 1] = streaming_attention(qh, kh, vh, int(p1), int(p2), acc=acc)
        elif ty == "block_sparse":
            idx, cnt = select_block_sparse_topk_indices(qh, kh, int(p1), dtype)
            sel[h] = (idx, cnt)
            out[:, h:h + 1] = block_sparse_from_indices(qh, kh, vh, idx, acc=acc)
        elif ty == "dense":
            out[:, h:h + 1] = dense_causal(qh, kh, vh, acc=acc)
        else:
            raise ValueError(f"unsupported pattern {ty!r}")
    return out, sel


# ---------------------------------------------------------------------------
# algorithmic work (D unpadded)
# ---------------------------------------------------------------------------
def stream_pairs(s: int, n_init: int, n_local: int) -> int:
    """Visible (query, key) pairs of one stream_llm head with S_q = S_k = s."""
    i = np.arange(s, dtype=np.int64)
    lo = np.maximum(0, i - n_local + 1)
    return int(((i - lo + 1) + np.minimum(n_init, lo)).sum())


def block_tiles(s: int, topk: int) -> int:
    """Computed 64x64 tiles of one block_sparse head: sum_bq min(k, bq+1)."""
    n_b = -(-s // BLOCK)
    k = min(topk, n_b)
    bq = np.arange(n_b, dtype=np.int64)
    return int(np.minimum(k, bq + 1).sum())


def causal_pairs(s: int) -> int:
    return s * (s + 1) // 2
