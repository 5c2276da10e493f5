// Kernel parameter blocks and launchers shared by the C ABI (msa_abi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "msa_common.h"

namespace msa {

// Pooled Q and K of the block estimator, in the input dtype (the pooled
// values are the reference's bf16/fp16 means, so 16 bits hold them exactly):
//   q_pool [batch*n_slots][n_qb_pad][D]  (rows n_qb .. n_qb_pad-1 unused)
//   k_pool [batch*n_slots][n_kb][D]      (entry b * n_slots + i: the i-th
//                                         distinct kv head of the slots)
// Blocks per pooling workgroup: one thread per (block, 16-byte chunk of a
// row), 16 blocks up to D = 128, 8 at D = 256, 4 at D = 512.
__host__ __device__ constexpr int pool_blocks_for(int D) { return D > 256 ? 4 : D > 128 ? 8 : 16; }

struct PoolParams {
  const void* q;
  const void* k;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t s_q, s_k;
  int n_qb, n_kb, n_qb_pad;  // n_qb_pad: n_qb rounded up to kScoreRowPad
  int pool_rows;             // rows per pooled block: 64, 128, 256 or 512
  int pool_blocks;           // blocks per pooling workgroup: pool_blocks_for(D)
  int batch, n_slots, kv_group;
  int n_kvp;                 // distinct kv heads of the slots
  uint16_t* q_pool;
  uint16_t* k_pool;
  int16_t slot_heads[kMaxHeads];  // head of q for each slot (kernel-argument copy)
  int16_t kvp_head[kMaxHeads];    // kv head of each distinct pooled K entry
};

struct ScoreParams {
  const uint16_t* q_pool;  // [batch*n_slots][n_qb_pad][D]
  const uint16_t* k_pool;  // [batch*n_slots][n_kb][D]
  float* scores;  // [batch*n_slots][n_qb_pad][n_kb_pad]: approximate pooled scores; the
                  // selection keeps its per-row keys there when they do not fit registers
  int32_t* idx;  // [batch*n_slots][n_qb][topk_max]
  int32_t* cnt;  // [batch*n_slots][n_qb]
  int n_qb, n_kb, n_qb_pad, n_kb_pad, topk_max, batch, n_slots;
  int s_q, s_k;  // row i of the query is absolute position s_k - s_q + i
  int block;     // tokens per block (the pooling's rows)
  float scale;
  int flags;     // kSelectForceFirst | kSelectForceDiag
  int16_t slot_topk[kMaxHeads];
  int16_t slot_kvp[kMaxHeads];  // pooled K entry of each slot
};

// Selector options: block 0 / the query block's own (diagonal, q-frame)
// block always selected, inside the top-k (their scores count as +inf; ties
// among forced ids go to the lower id).
constexpr int kSelectForceFirst = 1;
// Pooled-Q rows are padded to a multiple of the scoring row group; score
// rows to a multiple of 16 candidates (16-byte aligned quads).
constexpr int kScoreRowPad = 16;
constexpr int kSelectForceDiag = 2;

// 32-bit fields throughout: the kernel reads these with scalar loads, which
// have no 16-bit form on gfx950.
struct HeadArg {
  int32_t kind;
  int32_t slot;
  int32_t p1;  // stream: n_init
  int32_t p2;  // stream: n_local
  float scale_log2;  // softmax scale * log2(e)
};

struct AttnParams {
  const void* q;
  const void* k;
  const uint16_t* kt;  // staged K operands (stage_kernel; unused when k_in_place)
  const uint16_t* vt;  // staged V operands (stage_kernel)
  void* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t o_sb, o_sh, o_ss;
  int batch, heads, kv_group, s_q, s_k, n_qb, n_kb, s_pad;
  // 1: the QK operands are read from k's own rows (every operand load is 16
  // rows x 64 contiguous bytes) instead of the staged kt (see k_in_place)
  int k_in_place;
  const int32_t* idx;
  const int32_t* cnt;
  int idx_slots, topk_max;
  // Work items of this launch.  n_hl > 0: the items are (head_order[hl],
  // query block) for hl < n_hl, listed head-major with query blocks
  // longest-first; XCD x (workgroup i with i % 8 == x) takes items
  // xcd_start[x] + (i / 8) for i / 8 < xcd_count[x].  n_hl == 0: every
  // (batch, head) pair of the layer in plain order.
  int n_hl;
  int xcd_start[8];
  int xcd_count[8];
  int* queue;      // 8 counters of the XCD ranges (zeroed before each launch)
  int wg_per_xcd;  // CUs per XCD
  // vertical_and_slash launch: per (b * vs_slots + slot, query block) and
  // wave w (the 16-key chunk [16w, 16w+16) of every tile) a list of vs_cap
  // entries (tile id << 16 | the chunk's 16 key bits; gathered vertical
  // tiles as n_kb + g) holding only the tiles whose chunk has a visible key,
  // and its (unmasked prefix, total) counts; gathered vertical operands per
  // slot in stage_kernel's layout, nv_pad keys each.
  const uint32_t* vs_lists;  // [row][4][vs_cap]
  const int32_t* vs_cnt;     // [row][4][2]
  const uint16_t* gkt;
  const uint16_t* gvt;
  int vs_slots, vs_cap, nv_pad;
  const int32_t* vexp;  // [batch * kv_heads]: staged V = V * 2^-vexp (stage_kernel)
  int32_t head_order[kMaxHeads];
  HeadArg hd[kMaxHeads];
};
static_assert(sizeof(AttnParams) <= 4096, "attention kernel arguments exceed 4 KB");

// vertical_and_slash tile lists of one layer (vs_build_kernel).
struct VsBuildParams {
  const int32_t* v_idx;  // [batch*slots][v_stride]: vertical columns, ascending, distinct
  const int32_t* v_cnt;  // [batch*slots]
  const int32_t* s_idx;  // [batch*slots][s_stride]: slash offsets, any order
  const int32_t* s_cnt;  // [batch*slots]
  uint32_t* lists;       // outputs in the AttnParams vs_* layout
  int32_t* cnt;
  int v_stride, s_stride, cap, n_qb, n_kb, s_k;
};

// vertical_and_slash estimator of a layer (vs_*_kernel): slot s is head
// slot_heads[s]; S_q == S_k == s.
struct VsEstParams {
  const void* q;
  const void* k;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int batch, kv_group, s, n_rows, n_slots, s_pad;
  float sqrt_d;       // fp32(sqrt(D)), the divisor of the scores
  uint16_t* x;        // [batch*slots][64][s_pad]: scores in the input dtype, -inf masked
  float* rmax;        // [batch*slots][64]
  double* rsum;       // [batch*slots][64]
  float* vert;        // [batch*slots][s]
  float* slash;       // [batch*slots][s]
  int32_t* v_idx;     // [batch*slots][v_stride]
  int32_t* v_cnt;     // [batch*slots]
  int32_t* s_idx;     // [batch*slots][s_stride]
  int32_t* s_cnt;     // [batch*slots]
  int v_stride, s_stride;
  int16_t slot_heads[kMaxHeads];
  int32_t slot_vsize[kMaxHeads];
  int32_t slot_ssize[kMaxHeads];
};

// Longest key axis of a vertical_and_slash head (the tile-list builder keeps
// one 64-bit mask per key tile in LDS).
constexpr int kVsMaxSeq = 131072;

struct StageParams {
  const void* k;
  const void* v;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  uint16_t* kt;  // [batch*kv_heads][s_pad/16][D/32][64][8] QK A operands (input dtype)
  uint16_t* vt;  // [batch*kv_heads][s_pad/16][D/32][64][8] PV A operands (fp16)
  int batch, kv_heads, s_k, s_pad;
  // plain mode: 1 stages V and K; 0 V only (the attention kernel reads K in
  // place); 2 K only (no V maxima: the V staging has run)
  int stage_k;
  // Gather mode (rows != nullptr): blockIdx.y = b * n_slots + slot; staged key
  // j of that slot is row rows[(b * n_slots + slot) * rows_stride + j] of kv
  // head slot_kvh[slot] for j < rows_cnt[b * n_slots + slot], zero after;
  // s_pad keys per slot.
  const int32_t* rows;
  const int32_t* rows_cnt;
  int rows_stride, n_slots;
  // V range handling.  Plain mode: every V tile writes the largest finite |V|
  // it holds to tmax[b * kv_heads + kvh][tile] (s_pad / 64 tiles); then
  // vscale_kernel sets vexp[b * kv_heads + kvh] = e, the smallest e >= 0 with
  // max |V| * 2^-e <= 65504, and restages the head's V times 2^-e when e > 0
  // (exact for normal results).  Gather mode stages V times 2^-vexp of the
  // slot's kv head.  The attention kernel multiplies its output by 2^e.
  float* tmax;
  int32_t* vexp;
  int16_t slot_kvh[kMaxHeads];
  // Fused pooling (plain mode): the first n_pool_wg workgroups of the launch
  // run the block estimator's pooling pass with these parameters.
  int n_pool_wg;
  PoolParams pool;
};

struct DecodeParams {
  const void* q;  // [batch][heads][1][D]
  const void* k;  // [batch][kv_heads][s_k][D]
  const void* v;
  void* o;        // [batch][heads][1][D]
  int64_t q_sb, q_sh;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh;
  int batch, heads, kv_group, s_k;
  int n_split, chunk;  // key range of split s: [s*chunk, min((s+1)*chunk, s_k))
  float scale_log2;    // softmax scale * log2(e)
  float* part;         // workspace [batch*heads][n_split][D]: unnormalised O per split
  float* ml;           // workspace [batch*heads][n_split][2]: (m, l) per split
};

// Rotary embedding of one layer's q and k heads (rope_kernel).  q/k/qo/ko
// strides are [B][H][S][D] element strides; cos/sin are [B or 1][S][rot]
// (c_sb / n_sb = 0 broadcasts one table over the batch).  n_pair = rot / 16
// chunk pairs and n_pass = (D - rot) / 8 copied chunks per head row.
struct RopeParams {
  const void* q;
  const void* k;
  const void* cos;
  const void* sin;
  void* qo;
  void* ko;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t qo_sb, qo_sh, qo_ss;
  int64_t ko_sb, ko_sh, ko_ss;
  int64_t c_sb, c_ss, n_sb, n_ss;
  int batch, heads, kv_heads, s, rot, half, n_pair, n_pass;
};

// Widest rotary part msa_rope_qk takes (its cos/sin rows are staged in LDS).
constexpr int kRopeMaxRot = 256;

// Most splits a decode call uses (one head alone gets this many).
constexpr int kDecodeMaxSplit = 2048;

hipError_t launch_pool(const PoolParams& p, int dtype, int D, hipStream_t st);
int pool_workgroups(const PoolParams& p);
hipError_t launch_score(const ScoreParams& p, int dtype, int D, hipStream_t st);
int score_rows_for(int n_kb);
hipError_t launch_stage(const StageParams& p, int dtype, int D, hipStream_t st);
hipError_t launch_vscale(const StageParams& p, int dtype, int D, hipStream_t st);
hipError_t launch_decode(const DecodeParams& p, int dtype, int out_dtype, int D, hipStream_t st);
hipError_t launch_attention(const AttnParams& p, int dtype, int out_dtype, int D,
                            hipStream_t st);
hipError_t launch_attention_vs(const AttnParams& p, int dtype, int out_dtype, int D,
                               hipStream_t st);
hipError_t launch_vs_build(const VsBuildParams& p, int n_bs, hipStream_t st);
hipError_t launch_vs_estimate(const VsEstParams& p, int dtype, int D, hipStream_t st);
hipError_t launch_rope(const RopeParams& p, int dtype, hipStream_t st);

}  // namespace msa
