/*
 * msa.h — C ABI of the MI355X sparse prefill attention library (libmsa.so).
 *
 * The reference (white-jim/MInference-NPU) exposes this path only as Python
 * functions; it has no FFI.  Each entry point below replaces one of those
 * Python call sites and is bound from Python through ctypes
 * (minference-npu_amd/minference/_abi.py).  Paths below are relative to
 * MInference-NPU/ in the reference tree.
 *
 * Conventions
 *   - Every tensor pointer is a DEVICE pointer; the caller owns every buffer.
 *     The library allocates nothing and never synchronises the stream.
 *   - Tensors are 4-D [B, H, S, D] views described by msa_tensor4 (strides in
 *     elements).  The innermost (D) stride must be 1 and rows must be 16-byte
 *     aligned, so the HF BNSD views of a fused qkv projection are read in place.
 *   - Return value: 0 = launched; negative MSA_E_* = host-side validation
 *     failed and nothing was launched; positive = hipError_t reported by the
 *     runtime right after the launch.
 *   - Calls on the same stream are ordered; calls that share a workspace on
 *     different streams race.
 */
#ifndef MSA_H_
#define MSA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSA_ABI_VERSION 12

/* status codes (negative: validation, nothing launched) */
#define MSA_OK 0
#define MSA_E_NULL (-1)        /* a required pointer is NULL */
#define MSA_E_RANK (-2)        /* shape mismatch between q/k/v/o */
#define MSA_E_DTYPE (-3)       /* unsupported or mismatched dtype */
#define MSA_E_HEAD_DIM (-4)    /* D not in {64, 96, 128, 256, 512} ({64, 96, 128} for vertical_and_slash) */
#define MSA_E_ALIGN (-5)       /* D stride != 1, rows not 16-byte aligned or row stride >= 2^24 */
#define MSA_E_BLOCK (-6)       /* unsupported block size */
#define MSA_E_TOPK (-7)        /* topk < 1 or topk > n_kv_blocks */
#define MSA_E_HEADS (-8)       /* bad head count / head index / kind */
#define MSA_E_WORKSPACE (-9)   /* workspace missing or too small */
#define MSA_E_SEQ (-10)        /* S_q > S_k (causal kinds), S_q == 0, or too long */
#define MSA_E_SLOTS (-11)      /* sparse head without an index slot, or bad index lists */
#define MSA_E_SCRATCH (-12)    /* more than the fixed scratch of a no-allocation entry point */
#define MSA_E_FLAGS (-13)      /* unknown flags, or flags that exclude each other */

/* element types */
#define MSA_DTYPE_BF16 1
#define MSA_DTYPE_FP16 2
#define MSA_DTYPE_FP32 3

/* head kinds (pattern names of the per-head JSON) */
#define MSA_KIND_DENSE 0  /* "dense"        */
#define MSA_KIND_STREAM 1 /* "stream_llm"   */
#define MSA_KIND_BLOCK 2  /* "block_sparse" */
#define MSA_KIND_VS 3     /* "vertical_and_slash" */
#define MSA_KIND_FULL 4   /* dense without the causal mask (dense_attention(causal=False)) */
#define MSA_KIND_SKIP 5   /* left to another launch: rows neither read nor written */

/* msa_block_estimate_ex flags */
#define MSA_SELECT_FORCE_FIRST 1   /* block 0 always selected */
#define MSA_SELECT_FORCE_DIAG 2    /* the query block's own block always selected */
#define MSA_ESTIMATE_POOL_ONLY 4   /* phase 1 only: pooled Q and K into the workspace */
#define MSA_ESTIMATE_SELECT_ONLY 8 /* phase 2 only: scores and top-k from that workspace */

#define MSA_VS_MAX_SEQ 131072 /* longest S of a vertical_and_slash head */

#define MSA_MAX_HEADS 128 /* head descriptors per msa_layer_attention call */
#define MSA_BLOCK 64      /* tile of the attention kernels; estimator blocks are multiples of it */

typedef struct msa_tensor4 {
  void* data;
  int64_t size[4];   /* B, H, S, D (D = 64, 96, 128, 256 or 512) */
  int64_t stride[4]; /* elements */
  int32_t dtype;     /* MSA_DTYPE_* */
  int32_t reserved;
} msa_tensor4;

/* One attention head of a layer.
 *   kind   = MSA_KIND_*
 *   p1, p2 = stream_llm: n_init, n_local;  block_sparse: topk (unused here), 0;
 *            vertical_and_slash: vertical and slash counts (work estimate only)
 *   slot   = block_sparse: row of idx/cnt written by msa_block_estimate; else -1
 *   scale  = softmax scale applied to q.k, as the calling op defines it (the
 *            reference ops use different conventions, e.g. a padded head dim)
 * Mirrors the per-head record [type, p1, p2, score] parsed at
 * minference/modules/minference_forward.py:187-198, 404-419. */
typedef struct msa_head_desc {
  int32_t kind;
  int32_t p1;
  int32_t p2;
  int32_t slot;
  float scale;
  int32_t reserved;
} msa_head_desc;

typedef struct ihipStream_t* msa_stream_t; /* == hipStream_t */

int msa_abi_version(void);
const char* msa_status_str(int status);

/* Bytes of workspace msa_block_estimate needs: pooled Q and K in the input
 * dtype and the pooled scores of every row, fp32 (quadratic in S: 64 MiB per
 * slot at S = 64K, 1 GiB per slot at S = 2^18; the long-sequence limit is
 * S_k <= 2^20). */
size_t msa_estimate_workspace_bytes(int64_t batch, int32_t n_slots, int64_t s_q,
                                    int64_t s_k, int32_t head_dim);

/* Block top-k estimator for the block_sparse heads of a layer (one call for
 * all of them).  Replaces _select_block_sparse_topk_indices
 * (minference/ops/block_sparse_kernel_npu.py:230-263): block-token mean
 * pooling of Q and K in the input dtype (rounded to it; block = a multiple
 * of 64 tokens, the reference's block_size; ids, n_qb and n_kv_blocks are in
 * those blocks), fp32 pooled scores
 * q_pool.k_pool * score_scale, block-causal mask in the q-block frame, top-k
 * per query block, ids sorted ascending.  Ties break to the lower block id.
 *   slot_heads[s] (host array) = head index in q for slot s, s < n_slots
 *   slot_topk[s]  (host array or NULL = all topk_max) = top-k of slot s,
 *                 1 <= slot_topk[s] <= topk_max <= n_kv_blocks (the caller
 *                 clamps topk_blocks to n_kv_blocks as the reference does)
 *   idx  [B][n_slots][n_qb][topk_max] int32 (device): the first
 *        c = min(topk, bq+1) entries are the selected block ids ascending,
 *        entries c..topk-1 are the next ids bq+1, bq+2, ... (the reference's
 *        -inf picks in the q-block frame), entries topk..topk_max-1 are left
 *        untouched
 *   cnt  [B][n_slots][n_qb] int32 (device): how many leading entries any row
 *        of query block bq may attend under the absolute token-causal mask
 *        (row i at S_k - S_q + i): c, plus the surplus ids at or before the
 *        block's last row when S_q < S_k (reference
 *        minference/ops/block_sparse_kernel_npu.py:279-314) */
int msa_block_estimate(const msa_tensor4* q, const msa_tensor4* k,
                       const int32_t* slot_heads, const int32_t* slot_topk,
                       int32_t n_slots, int32_t block, int32_t topk_max,
                       float score_scale, int32_t* idx, int32_t* cnt,
                       void* workspace, size_t workspace_bytes,
                       msa_stream_t stream);

/* msa_block_estimate with selection flags (MSA_SELECT_*; 0 = the reference
 * selector, identical to msa_block_estimate).  FORCE_FIRST / FORCE_DIAG keep
 * block 0 / block bq (the query block's own, q-block frame) in every row's
 * selection, inside the top-k: forced ids rank above every scored id, and
 * between the two the lower id wins (top-k 1 with both flags keeps block 0).
 * The reference selector has no such option; it serves selection rules that
 * always keep the diagonal and first block.
 * The estimator is two passes (pooling, then scoring + top-k); POOL_ONLY and
 * SELECT_ONLY (one of them at a time) launch one pass, so a caller can run
 * the pooling first and the selection beside other work.  A SELECT_ONLY call
 * reads the pooled Q and K that a POOL_ONLY call with the same arguments left
 * in the same workspace (and block), and must be ordered after it (same
 * stream, or an event); a POOL_ONLY call leaves idx and cnt untouched.  Same counterpart
 * as msa_block_estimate
 * (minference/ops/block_sparse_kernel_npu.py:230-263). */
int msa_block_estimate_ex(const msa_tensor4* q, const msa_tensor4* k,
                          const int32_t* slot_heads, const int32_t* slot_topk,
                          int32_t n_slots, int32_t block, int32_t topk_max,
                          float score_scale, int32_t flags, int32_t* idx,
                          int32_t* cnt, void* workspace, size_t workspace_bytes,
                          msa_stream_t stream);

/* Bytes of workspace msa_layer_attention needs: K and V staged once per
 * layer in MFMA operand order (V as fp16, scaled per kv head by a power of
 * two when its magnitude exceeds the fp16 range, with the exponent kept in
 * the workspace and undone at the output; Inf and NaN pass through). */
size_t msa_attention_workspace_bytes(int64_t batch, int64_t kv_heads, int64_t s_k,
                                     int32_t head_dim);

/* All heads of one layer in one attention launch (plus one V staging launch).
 * Replaces the grouped dispatch of minference/modules/minference_forward.py:398-487
 * and the three ops it calls:
 *   streaming_forward       minference/ops/streaming_kernel_npu.py:349-397
 *   block_sparse attention  minference/ops/block_sparse_kernel_npu.py:441-601
 *   dense_attention         minference/backend_npu/attention.py:192-255
 * heads[h] (host array, n_heads == H of q) describes head h.  idx/cnt are the
 * msa_block_estimate outputs (or caller-built lists sorted ascending; entries
 * outside [0, n_kv_blocks), repeated or in the causal future are skipped);
 * they may be NULL when no head is block_sparse.  o may be bf16/fp16 (== q's
 * dtype) or fp32.  Rows with no visible key are written as 0.
 * MSA_KIND_FULL heads see every key (dense_attention(causal=False),
 * minference/backend_npu/attention.py:221-230); S_q > S_k is accepted only
 * when every head is MSA_KIND_FULL (or MSA_KIND_SKIP).  MSA_KIND_SKIP heads
 * are left out of the launch: their output rows are not written, their
 * descriptors' other fields are not read. */
int msa_layer_attention(const msa_tensor4* q, const msa_tensor4* k,
                        const msa_tensor4* v, const msa_tensor4* o,
                        const msa_head_desc* heads, int32_t n_heads,
                        const int32_t* idx, const int32_t* cnt, int32_t idx_slots,
                        int32_t topk_max, void* workspace, size_t workspace_bytes,
                        msa_stream_t stream);

/* The two launches msa_layer_attention makes, callable separately (so a
 * caller can time the attention kernel alone, or reuse one staging):
 *   msa_stage_kv: V [B][H_kv][S_k][D] -> MFMA operand order in the
 *                workspace (msa_attention_workspace_bytes bytes), and K too
 *                when the attention kernel cannot read it in place (rows
 *                that overlap, row stride < D, or one kv head's padded rows
 *                spanning more than 2^31 bytes); k and v have the same shape
 *                and dtype;
 *   msa_layer_attention_staged: same arguments and checks as
 *                msa_layer_attention, reads V (and K where it was staged)
 *                from the workspace msa_stage_kv wrote on the same stream,
 *                and K in place from k otherwise: k and v must be the views
 *                msa_stage_kv received.
 * Same reference counterpart as msa_layer_attention. */
int msa_stage_kv(const msa_tensor4* k, const msa_tensor4* v, void* workspace,
                 size_t workspace_bytes, msa_stream_t stream);
int msa_layer_attention_staged(const msa_tensor4* q, const msa_tensor4* k,
                               const msa_tensor4* v, const msa_tensor4* o,
                               const msa_head_desc* heads, int32_t n_heads,
                               const int32_t* idx, const int32_t* cnt,
                               int32_t idx_slots, int32_t topk_max, void* workspace,
                               size_t workspace_bytes, msa_stream_t stream);

/* msa_stage_kv and the pooling pass of the block estimator in one launch, for
 * the layer schedule of a layer with block_sparse heads:
 *   msa_stage_kv_pool (K/V staging + Q/K pooling) -> msa_block_estimate_ex
 *   (MSA_ESTIMATE_SELECT_ONLY, same estimator workspace) ->
 *   msa_layer_attention_staged, all on one stream.
 * q, k, slot_heads and n_slots are those of the msa_block_estimate_ex call
 * that follows; est_workspace is its workspace (msa_estimate_workspace_bytes),
 * workspace the attention workspace (msa_attention_workspace_bytes).
 * n_slots = 0 stages only (q, slot_heads and est_workspace unused).
 * Replaces the same calls as msa_stage_kv and the pooling step of
 * _select_block_sparse_topk_indices
 * (minference/ops/block_sparse_kernel_npu.py:240-252). */
int msa_stage_kv_pool(const msa_tensor4* q, const msa_tensor4* k, const msa_tensor4* v,
                      const int32_t* slot_heads, int32_t n_slots, void* est_workspace,
                      size_t est_workspace_bytes, void* workspace, size_t workspace_bytes,
                      msa_stream_t stream);


/* vertical_and_slash index lists of a layer: one slot per vertical_and_slash
 * head (msa_head_desc.slot).  Device arrays:
 *   v_idx [B][n_slots][v_stride]: vertical columns, ascending, distinct, in
 *         [0, S_k); the first v_cnt[b][slot] entries are used
 *   s_idx [B][n_slots][s_stride]: slash offsets s (the diagonal key = row - s),
 *         any order and range; the first s_cnt[b][slot] entries are used
 * These are the v_idx / s_idx of the reference's
 * vertical_slash_sparse_attention (minference/ops/vertical_slash_kernel_npu.py:
 * 518-525), with per-row counts.  Every head sharing a slot must read the
 * same kv head. */
typedef struct msa_vs_lists {
  const int32_t* v_idx;
  const int32_t* v_cnt;
  const int32_t* s_idx;
  const int32_t* s_cnt;
  int32_t n_slots;
  int32_t v_stride;
  int32_t s_stride;
  int32_t reserved;
} msa_vs_lists;

/* Bytes of workspace msa_vs_estimate needs (last-rows scores, row
 * statistics, column and diagonal sums). */
size_t msa_vs_estimate_workspace_bytes(int64_t batch, int32_t n_slots, int64_t s,
                                       int32_t head_dim);

/* vertical_and_slash estimator for the vertical_and_slash heads of a layer
 * (one call for all of them).  Replaces the index estimation of
 * _vertical_and_slash_kernel, minference/modules/minference_forward.py:
 * 140-165: scores of the last min(64, S) query rows in the input dtype,
 * divided by sqrt(D) and rounded again, causal within the last rows, fp64
 * softmax, column sums (first 30 forced) and diagonal sums (last 100
 * forced), top-k with ties to the lower index.
 *   slot_heads[s] (host) = head of q for slot s
 *   slot_vsize[s], slot_ssize[s] (host) = vertical / slash counts, already
 *     clamped as the reference does (min(S, max(v, 30)), min(S, max(s, 50)));
 *     1 <= size <= v_stride / s_stride
 *   v_idx [B][n_slots][v_stride], v_cnt [B][n_slots] (device): columns
 *     ascending, count = slot_vsize
 *   s_idx [B][n_slots][s_stride], s_cnt [B][n_slots] (device): slash offsets
 *     S - 1 - t descending, count = slot_ssize
 * These are exactly the msa_vs_lists msa_layer_attention_ex takes.  Needs
 * S_q == S_k <= MSA_VS_MAX_SEQ. */
int msa_vs_estimate(const msa_tensor4* q, const msa_tensor4* k, const int32_t* slot_heads,
                    const int32_t* slot_vsize, const int32_t* slot_ssize, int32_t n_slots,
                    int32_t* v_idx, int32_t* v_cnt, int32_t v_stride, int32_t* s_idx,
                    int32_t* s_cnt, int32_t s_stride, void* workspace, size_t workspace_bytes,
                    msa_stream_t stream);

/* Bytes of the vertical_and_slash workspace of msa_layer_attention_ex: the
 * per-(slot, query block) tile lists with their key masks, and the vertical
 * columns' K and V staged contiguously per slot. */
size_t msa_vs_workspace_bytes(int64_t batch, int32_t n_slots, int64_t s_k, int32_t v_stride,
                              int32_t head_dim);

/* msa_layer_attention with vertical_and_slash heads (kind MSA_KIND_VS).
 * Replaces, besides msa_layer_attention's counterparts, the
 * vertical_and_slash group of minference/modules/minference_forward.py:421-436
 * and vertical_slash_sparse_attention
 * (minference/ops/vertical_slash_kernel_npu.py:518-599): visibility of
 * _build_vs_mask_direct (:282-367) under the causal mask, as one tile-list
 * build launch, one gather of the vertical columns and one attention launch
 * for the vertical_and_slash heads (the other heads keep their own launch).
 * vertical_and_slash heads need S_q == S_k <= MSA_VS_MAX_SEQ and
 * B * H <= MSA_MAX_HEADS.  vs and vs_workspace may be NULL when no head is
 * vertical_and_slash.  stage = 0 reads what msa_stage_kv staged for the
 * same k and v (as msa_layer_attention_staged), 1 stages first. */
int msa_layer_attention_ex(const msa_tensor4* q, const msa_tensor4* k, const msa_tensor4* v,
                           const msa_tensor4* o, const msa_head_desc* heads, int32_t n_heads,
                           const int32_t* idx, const int32_t* cnt, int32_t idx_slots,
                           int32_t topk_max, const msa_vs_lists* vs, void* vs_workspace,
                           size_t vs_workspace_bytes, void* workspace, size_t workspace_bytes,
                           int32_t stage, msa_stream_t stream);

/* Decode: one query row per head (q [B][H][1][D]) against the whole cache
 * (k, v [B][H_kv][S_k][D], any strides with D contiguous and 16-byte rows),
 * every key visible.  Replaces decode_dense,
 * minference/backend_npu/attention.py:274-314, which the patched forward
 * calls for q_len == 1 (minference/modules/minference_forward.py:488-490).
 * scale is the softmax scale (the reference default is 1/sqrt(D)).  o may be
 * q's dtype or fp32.  Two launches (split-K partials, then their merge); the
 * workspace holds the partials (msa_decode_workspace_bytes). */
size_t msa_decode_workspace_bytes(int64_t batch, int64_t heads, int64_t s_k, int32_t head_dim);
int msa_decode_attention(const msa_tensor4* q, const msa_tensor4* k, const msa_tensor4* v,
                         const msa_tensor4* o, float scale, void* workspace,
                         size_t workspace_bytes, msa_stream_t stream);

/* msa_decode_attention without a workspace argument: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * split-K partials go to a fixed per-GPU device array of
 * MSA_DECODE_SCRATCH_BYTES inside the library (held by each GPU it runs on
 * until the process ends); the call allocates nothing.  A call whose partials
 * would not fit (msa_decode_workspace_bytes > MSA_DECODE_SCRATCH_BYTES; at
 * D = 128 that is B * H above about 7800) returns MSA_E_SCRATCH.  Every call
 * on one GPU shares that array: calls that overlap on one GPU (different
 * streams, or host threads without ordering) race.  Same arguments, checks
 * and results as msa_decode_attention. */
#define MSA_DECODE_SCRATCH_BYTES (4u << 20)
int msa_decode_attention_noalloc(const msa_tensor4* q, const msa_tensor4* k,
                                 const msa_tensor4* v, const msa_tensor4* o, float scale,
                                 msa_stream_t stream);

/* Rotary position embedding of one layer's query and key heads, one launch.
 * Replaces the apply_rotary_pos_emb call of the patched forward
 * (minference/modules/minference_forward.py:336-341, HF's rotate-half RoPE):
 *   out[:rot/2]    = q[:rot/2] * cos[:rot/2] - q[rot/2:rot] * sin[:rot/2]
 *   out[rot/2:rot] = q[rot/2:rot] * cos[rot/2:] + q[:rot/2] * sin[rot/2:]
 *   out[rot:]      = q[rot:]                       (partial rotary)
 * with every product and sum rounded to the input dtype as the eager
 * elementwise ops round them, so the result is bit-identical to
 * q * cos + rotate_half(q) * sin.  Same for k.
 *   q [B][H][S][D], k [B][H_kv][S][D]: views (e.g. of a fused qkv projection)
 *   cos, sin [B or 1][1][S][rot]: the position tables (a batch size of 1
 *     broadcasts); rot % 16 == 0, rot <= min(D, 256), D % 8 == 0, D <= 512
 *   q_out, k_out: same shapes; may be q / k themselves (in place), must not
 *     overlap them otherwise
 * All bf16 or all fp16, D contiguous, 16-byte aligned rows. */
int msa_rope_qk(const msa_tensor4* q, const msa_tensor4* k, const msa_tensor4* cos,
                const msa_tensor4* sin, const msa_tensor4* q_out, const msa_tensor4* k_out,
                msa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MSA_H_ */
