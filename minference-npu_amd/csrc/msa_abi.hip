// C ABI (include/msa.h): host-side validation, argument packing and launches.
// Nothing here allocates device memory or synchronises the stream.

#include <math.h>

#include <algorithm>
#include <mutex>
#include <string.h>

#include "../../include/msa.h"
#include "msa_kernels.h"

using namespace msa;

namespace {

constexpr int64_t kMaxSeq = int64_t(1) << 20;  // 1M tokens: 16384 blocks
constexpr size_t kQueueBytes = 256;             // work-queue counters of an attention launch

int elem_size(int dtype) {
  switch (dtype) {
    case MSA_DTYPE_BF16:
    case MSA_DTYPE_FP16: return 2;
    case MSA_DTYPE_FP32: return 4;
    default: return 0;
  }
}

bool head_dim_ok(int64_t d) { return d == 64 || d == 96 || d == 128 || d == 256 || d == 512; }
// vertical_and_slash estimator and attention: up to 128
bool vs_head_dim_ok(int64_t d) { return d == 64 || d == 96 || d == 128; }

// D contiguous, every row and the base 16-byte aligned, row stride below
// 2^24 elements (the attention kernel addresses a query block's 64 rows
// with 32-bit byte offsets).
bool aligned(const msa_tensor4* t) {
  const int es = elem_size(t->dtype);
  if (es == 0 || t->stride[3] != 1) return false;
  if (t->stride[2] < 0 || t->stride[2] >= (int64_t(1) << 24)) return false;
  if ((reinterpret_cast<uintptr_t>(t->data) & 15u) != 0) return false;
  for (int i = 0; i < 3; ++i)
    if (t->size[i] > 1 && ((t->stride[i] * es) & 15) != 0) return false;
  return true;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Typed pointer at a byte offset of a caller's workspace.
template <typename P>
P* ws_at(void* workspace, size_t off) {
  return reinterpret_cast<P*>(static_cast<unsigned char*>(workspace) + off);
}

int check_qk(const msa_tensor4* q, const msa_tensor4* k) {
  if (!q || !k || !q->data || !k->data) return MSA_E_NULL;
  for (int i = 0; i < 4; ++i)
    if (q->size[i] <= 0 || k->size[i] <= 0) return MSA_E_RANK;
  if (q->size[0] != k->size[0] || q->size[3] != k->size[3]) return MSA_E_RANK;
  if (q->size[1] % k->size[1] != 0) return MSA_E_RANK;
  if (q->dtype != k->dtype) return MSA_E_DTYPE;
  if (q->dtype != MSA_DTYPE_BF16 && q->dtype != MSA_DTYPE_FP16) return MSA_E_DTYPE;
  if (!head_dim_ok(q->size[3])) return MSA_E_HEAD_DIM;
  if (!aligned(q) || !aligned(k)) return MSA_E_ALIGN;
  if (q->size[2] > kMaxSeq || k->size[2] > kMaxSeq) return MSA_E_SEQ;
  return MSA_OK;
}

}  // namespace

extern "C" {

int msa_abi_version(void) { return MSA_ABI_VERSION; }

const char* msa_status_str(int status) {
  switch (status) {
    case MSA_OK: return "ok";
    case MSA_E_NULL: return "a required pointer is NULL";
    case MSA_E_RANK: return "shape mismatch between q, k, v and o";
    case MSA_E_DTYPE: return "unsupported or mismatched dtype (q/k/v must be bf16 or fp16; o same or fp32)";
    case MSA_E_HEAD_DIM: return "head_dim must be 64, 96, 128, 256 or 512 (vertical_and_slash: 64, 96 or 128)";
    case MSA_E_ALIGN: return "head_dim stride must be 1, rows 16-byte aligned and the row stride below 2^24";
    case MSA_E_BLOCK: return "block size must be a multiple of 64";
    case MSA_E_TOPK: return "topk must be in [1, n_kv_blocks]";
    case MSA_E_HEADS: return "bad head count, head index or head kind";
    case MSA_E_WORKSPACE: return "workspace missing or too small";
    case MSA_E_SEQ: return "sequence lengths must satisfy 0 < S_q <= S_k <= 2^20 (S_q > S_k only for full heads)";
    case MSA_E_SLOTS: return "sparse head without a valid index slot, or bad idx/cnt or vertical_and_slash lists";
    case MSA_E_SCRATCH: return "the call needs more than the fixed scratch of a no-allocation entry point (MSA_DECODE_SCRATCH_BYTES)";
    case MSA_E_FLAGS: return "unknown flags, or MSA_ESTIMATE_POOL_ONLY and MSA_ESTIMATE_SELECT_ONLY together";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}

}  // extern "C"

namespace {

// Estimator workspace: pooled Q [B*slots][n_qb_pad][D] and pooled K
// [B*slots][n_kb][D] (the slots' distinct kv heads) in the input dtype, then
// the approximate scores [B*slots][n_qb_pad][n_kb_pad] fp32.
struct EstLayout {
  int n_qb, n_kb, n_qb_pad, n_kb_pad;
  size_t q, k, sc, total;
};

EstLayout est_layout(int64_t batch, int64_t n_slots, int64_t s_q, int64_t s_k, int64_t D,
                     int64_t block = MSA_BLOCK) {
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  EstLayout L;
  L.n_qb = int(cdiv(s_q, block));
  L.n_kb = int(cdiv(s_k, block));
  L.n_qb_pad = int(cdiv(L.n_qb, kScoreRowPad) * kScoreRowPad);
  L.n_kb_pad = int(cdiv(L.n_kb, 16) * 16);
  const int64_t sb = batch * n_slots;
  L.q = 0;
  L.k = up(size_t(sb) * L.n_qb_pad * D * 2);
  L.sc = L.k + up(size_t(sb) * L.n_kb * D * 2);
  L.total = L.sc + up(size_t(sb) * L.n_qb_pad * L.n_kb_pad * 4);
  return L;
}

// Checks shared by the estimator entry points; fills the pooling parameters
// (slot -> distinct kv head entry in slot_kvp).
int pool_setup(const msa_tensor4* q, const msa_tensor4* k, const int32_t* slot_heads,
               int32_t n_slots, void* workspace, size_t workspace_bytes, PoolParams& pp,
               int16_t* slot_kvp, EstLayout& L, int block = MSA_BLOCK) {
  int st = check_qk(q, k);
  if (st != MSA_OK) return st;
  if (!slot_heads) return MSA_E_NULL;
  if (n_slots <= 0 || n_slots > kMaxHeads) return MSA_E_HEADS;
  const int H = int(q->size[1]);
  for (int s = 0; s < n_slots; ++s)
    if (slot_heads[s] < 0 || slot_heads[s] >= H) return MSA_E_HEADS;
  if (q->size[0] * n_slots > 65535) return MSA_E_HEADS;
  const int D = int(q->size[3]);
  L = est_layout(q->size[0], n_slots, q->size[2], k->size[2], D, block);
  if (score_rows_for(L.n_kb) == 0) return MSA_E_SEQ;
  if (!workspace || workspace_bytes < L.total) return MSA_E_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return MSA_E_ALIGN;
  memset(&pp, 0, sizeof(pp));
  pp.q = q->data;
  pp.k = k->data;
  pp.q_sb = q->stride[0]; pp.q_sh = q->stride[1]; pp.q_ss = q->stride[2];
  pp.k_sb = k->stride[0]; pp.k_sh = k->stride[1]; pp.k_ss = k->stride[2];
  pp.s_q = q->size[2];
  pp.s_k = k->size[2];
  pp.n_qb = L.n_qb;
  pp.n_kb = L.n_kb;
  pp.n_qb_pad = L.n_qb_pad;
  pp.pool_rows = block;
  pp.pool_blocks = pool_blocks_for(D);
  pp.batch = int(q->size[0]);
  pp.n_slots = n_slots;
  pp.kv_group = int(q->size[1] / k->size[1]);
  pp.q_pool = ws_at<uint16_t>(workspace, L.q);
  pp.k_pool = ws_at<uint16_t>(workspace, L.k);
  pp.n_kvp = 0;
  for (int s = 0; s < n_slots; ++s) {
    pp.slot_heads[s] = int16_t(slot_heads[s]);
    const int kvh = slot_heads[s] / pp.kv_group;
    int i = 0;
    while (i < pp.n_kvp && pp.kvp_head[i] != kvh) ++i;
    if (i == pp.n_kvp) pp.kvp_head[pp.n_kvp++] = int16_t(kvh);
    slot_kvp[s] = int16_t(i);
  }
  return MSA_OK;
}

}  // namespace

extern "C" {

size_t msa_estimate_workspace_bytes(int64_t batch, int32_t n_slots, int64_t s_q, int64_t s_k,
                                    int32_t head_dim) {
  if (batch <= 0 || n_slots <= 0 || s_q <= 0 || s_k <= 0 || head_dim <= 0) return 0;
  return est_layout(batch, n_slots, s_q, s_k, head_dim).total;
}

int msa_block_estimate(const msa_tensor4* q, const msa_tensor4* k, const int32_t* slot_heads,
                       const int32_t* slot_topk, int32_t n_slots, int32_t block,
                       int32_t topk_max, float score_scale, int32_t* idx, int32_t* cnt,
                       void* workspace, size_t workspace_bytes, msa_stream_t stream) {
  return msa_block_estimate_ex(q, k, slot_heads, slot_topk, n_slots, block, topk_max,
                               score_scale, 0, idx, cnt, workspace, workspace_bytes, stream);
}

int msa_block_estimate_ex(const msa_tensor4* q, const msa_tensor4* k, const int32_t* slot_heads,
                          const int32_t* slot_topk, int32_t n_slots, int32_t block,
                          int32_t topk_max, float score_scale, int32_t flags, int32_t* idx,
                          int32_t* cnt, void* workspace, size_t workspace_bytes,
                          msa_stream_t stream) {
  constexpr int32_t kKnown = MSA_SELECT_FORCE_FIRST | MSA_SELECT_FORCE_DIAG |
                              MSA_ESTIMATE_POOL_ONLY | MSA_ESTIMATE_SELECT_ONLY;
  if ((flags & ~kKnown) != 0) return MSA_E_FLAGS;
  const int32_t phase = flags & (MSA_ESTIMATE_POOL_ONLY | MSA_ESTIMATE_SELECT_ONLY);
  if (phase == (MSA_ESTIMATE_POOL_ONLY | MSA_ESTIMATE_SELECT_ONLY)) return MSA_E_FLAGS;
  flags &= MSA_SELECT_FORCE_FIRST | MSA_SELECT_FORCE_DIAG;
  int st = check_qk(q, k);
  if (st != MSA_OK) return st;
  if (block < MSA_BLOCK || block % MSA_BLOCK != 0 || block > kMaxSeq) return MSA_E_BLOCK;
  if (!slot_heads || !idx || !cnt) return MSA_E_NULL;
  if (n_slots <= 0 || n_slots > kMaxHeads) return MSA_E_HEADS;
  const int64_t n_kb_blk = cdiv(k->size[2], block);
  if (topk_max < 1 || topk_max > n_kb_blk) return MSA_E_TOPK;
  if (slot_topk)
    for (int s = 0; s < n_slots; ++s)
      if (slot_topk[s] < 1 || slot_topk[s] > topk_max) return MSA_E_TOPK;
  if (!(score_scale > 0.0f) || !isfinite(score_scale)) return MSA_E_TOPK;
  PoolParams pp;
  int16_t slot_kvp[kMaxHeads];
  EstLayout L;
  st = pool_setup(q, k, slot_heads, n_slots, workspace, workspace_bytes, pp, slot_kvp, L,
                  block);
  if (st != MSA_OK) return st;
  const int D = int(q->size[3]);

  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  if (phase != MSA_ESTIMATE_SELECT_ONLY) e = launch_pool(pp, q->dtype, D, hs);
  if (e != hipSuccess) return int(e);
  if (phase == MSA_ESTIMATE_POOL_ONLY) return MSA_OK;

  ScoreParams sp;
  memset(&sp, 0, sizeof(sp));
  sp.q_pool = pp.q_pool;
  sp.k_pool = pp.k_pool;
  sp.scores = ws_at<float>(workspace, L.sc);
  sp.idx = idx;
  sp.cnt = cnt;
  sp.n_qb = L.n_qb;
  sp.n_kb = L.n_kb;
  sp.n_qb_pad = L.n_qb_pad;
  sp.n_kb_pad = L.n_kb_pad;
  sp.topk_max = topk_max;
  sp.batch = int(q->size[0]);
  sp.n_slots = n_slots;
  sp.s_q = int(q->size[2]);
  sp.s_k = int(k->size[2]);
  sp.block = block;
  sp.scale = score_scale;
  sp.flags = flags;
  for (int s = 0; s < n_slots; ++s) {
    sp.slot_topk[s] = int16_t(slot_topk ? slot_topk[s] : topk_max);
    sp.slot_kvp[s] = slot_kvp[s];
  }
  e = launch_score(sp, q->dtype, D, hs);
  return e == hipSuccess ? MSA_OK : int(e);
}

// Attention workspace: staged V operands (fp16), staged K operands (input
// dtype; written only where the attention kernel cannot read K in place,
// see k_in_place), per-tile V maxima (fp32), per-head V exponents (int32),
// then the work-queue counters of the attention launch.
struct AttnLayout {
  size_t vt, kt, tmax, vexp, total;
};

static AttnLayout attn_layout(int64_t B, int64_t Hkv, int64_t Sk, int64_t D) {
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  const int64_t n_kb = cdiv(Sk, MSA_BLOCK);
  AttnLayout L;
  L.vt = 0;
  L.kt = size_t(B * Hkv * D * n_kb * MSA_BLOCK) * 2;
  L.tmax = L.kt * 2;
  L.vexp = up(L.tmax + size_t(B * Hkv * n_kb) * 4);
  L.total = up(L.vexp + size_t(B * Hkv) * 4) + kQueueBytes;
  return L;
}

size_t msa_attention_workspace_bytes(int64_t batch, int64_t kv_heads, int64_t s_k,
                                     int32_t head_dim) {
  if (batch <= 0 || kv_heads <= 0 || s_k <= 0 || head_dim <= 0) return 0;
  return attn_layout(batch, kv_heads, s_k, head_dim).total;
}

// work-queue counters at the end of the attention workspace
static int* queue_of(void* workspace, size_t workspace_bytes) {
  return reinterpret_cast<int*>(static_cast<unsigned char*>(workspace) + workspace_bytes -
                                kQueueBytes);
}

// CUs per XCD of the current device (8 XCDs on gfx950)
static int cus_per_xcd() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  return cus >= 8 ? cus / 8 : 1;
}


// The attention kernel reads K in place, from the caller's rows, when every
// offset of one kv head's padded rows fits 31 bits and the rows do not
// overlap; otherwise the staging writes K in operand order first.  D = 256
// and 512 always take staged K: their kernel reads every tile's K once per
// wave, and a staged operand is 8 whole cache lines where an in-place one
// touches 16 half lines.
static bool k_in_place(const msa_tensor4* k) {
  const int64_t D = k->size[3], ss = k->stride[2];
  const int64_t s_pad = cdiv(k->size[2], MSA_BLOCK) * MSA_BLOCK;
  return D <= 128 && ss >= D && (s_pad * ss + D) * 2 <= (int64_t(1) << 31);
}

static int stage_setup(const msa_tensor4* k, const msa_tensor4* v, void* workspace,
                       size_t workspace_bytes, StageParams& sp) {
  if (!k || !v || !k->data || !v->data) return MSA_E_NULL;
  for (int i = 0; i < 4; ++i) {
    if (v->size[i] <= 0) return MSA_E_RANK;
    if (k->size[i] != v->size[i]) return MSA_E_RANK;
  }
  if (v->dtype != MSA_DTYPE_BF16 && v->dtype != MSA_DTYPE_FP16) return MSA_E_DTYPE;
  if (k->dtype != v->dtype) return MSA_E_DTYPE;
  if (!head_dim_ok(v->size[3])) return MSA_E_HEAD_DIM;
  if (!aligned(v) || !aligned(k)) return MSA_E_ALIGN;
  if (v->size[2] > kMaxSeq) return MSA_E_SEQ;
  const int64_t B = v->size[0], Hkv = v->size[1], Sk = v->size[2];
  const int D = int(v->size[3]);
  if (B * Hkv > 65535) return MSA_E_HEADS;
  const size_t need = msa_attention_workspace_bytes(B, Hkv, Sk, D);
  if (!workspace || workspace_bytes < need) return MSA_E_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return MSA_E_ALIGN;
  memset(&sp, 0, sizeof(sp));  // gather-mode fields stay null: plain staging
  sp.k = k->data;
  sp.v = v->data;
  sp.k_sb = k->stride[0]; sp.k_sh = k->stride[1]; sp.k_ss = k->stride[2];
  sp.v_sb = v->stride[0]; sp.v_sh = v->stride[1]; sp.v_ss = v->stride[2];
  const AttnLayout L = attn_layout(B, Hkv, Sk, D);
  sp.vt = ws_at<uint16_t>(workspace, L.vt);
  sp.kt = ws_at<uint16_t>(workspace, L.kt);
  sp.tmax = ws_at<float>(workspace, L.tmax);
  sp.vexp = ws_at<int32_t>(workspace, L.vexp);
  sp.batch = int(B);
  sp.kv_heads = int(Hkv);
  sp.s_k = int(Sk);
  sp.s_pad = int(cdiv(Sk, MSA_BLOCK) * MSA_BLOCK);
  sp.stage_k = k_in_place(k) ? 0 : 1;
  return MSA_OK;
}

static int stage_launch(const StageParams& sp, int dtype, int D, hipStream_t hs) {
  hipError_t e = launch_stage(sp, dtype, D, hs);
  if (e == hipSuccess) e = launch_vscale(sp, dtype, D, hs);
  return e == hipSuccess ? MSA_OK : int(e);
}

int msa_stage_kv(const msa_tensor4* k, const msa_tensor4* v, void* workspace,
                 size_t workspace_bytes, msa_stream_t stream) {
  StageParams sp;
  const int st = stage_setup(k, v, workspace, workspace_bytes, sp);
  if (st != MSA_OK) return st;
  return stage_launch(sp, v->dtype, int(v->size[3]), reinterpret_cast<hipStream_t>(stream));
}

int msa_stage_kv_pool(const msa_tensor4* q, const msa_tensor4* k, const msa_tensor4* v,
                      const int32_t* slot_heads, int32_t n_slots, void* est_workspace,
                      size_t est_workspace_bytes, void* workspace, size_t workspace_bytes,
                      msa_stream_t stream) {
  StageParams sp;
  int st = stage_setup(k, v, workspace, workspace_bytes, sp);
  if (st != MSA_OK) return st;
  if (n_slots > 0) {
    int16_t slot_kvp[kMaxHeads];
    EstLayout L;
    st = pool_setup(q, k, slot_heads, n_slots, est_workspace, est_workspace_bytes, sp.pool,
                    slot_kvp, L);
    if (st != MSA_OK) return st;
    sp.n_pool_wg = pool_workgroups(sp.pool);
  } else if (n_slots < 0) {
    return MSA_E_HEADS;
  }
  return stage_launch(sp, v->dtype, int(v->size[3]), reinterpret_cast<hipStream_t>(stream));
}

// vertical_and_slash workspace: tile ids, key masks, counts per (slot,
// query block); gathered vertical K and V per slot.
struct VsLayout {
  int64_t n_rows;
  int cap, nv_pad;
  size_t lists, cnt, gk, gv, total;
};

static VsLayout vs_layout(int64_t B, int64_t n_slots, int64_t s_k, int64_t v_stride, int64_t D) {
  VsLayout L;
  const int64_t n_kb = cdiv(s_k, MSA_BLOCK);
  L.nv_pad = int(cdiv(std::max<int64_t>(v_stride, 1), MSA_BLOCK) * MSA_BLOCK);
  L.cap = int(n_kb + L.nv_pad / MSA_BLOCK);
  L.n_rows = B * n_slots * n_kb;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  size_t off = 0;
  L.lists = off;  // per row and wave: cap entries
  off = up(off + size_t(L.n_rows) * 4 * L.cap * 4);
  L.cnt = off;    // per row and wave: (unmasked, total)
  off = up(off + size_t(L.n_rows) * 4 * 2 * 4);
  L.gk = off;
  off = up(off + size_t(B * n_slots) * L.nv_pad * D * 2);
  L.gv = off;
  off = up(off + size_t(B * n_slots) * L.nv_pad * D * 2);
  L.total = off;
  return L;
}

// vertical_and_slash estimator workspace: scores, row max, row sums,
// column sums, diagonal sums.
struct VsEstLayout {
  size_t x, rmax, rsum, vert, slash, total;
};

static VsEstLayout vs_est_layout(int64_t B, int64_t n_slots, int64_t s) {
  VsEstLayout L;
  const int64_t s_pad = cdiv(s, MSA_BLOCK) * MSA_BLOCK;
  const int64_t bs = B * n_slots;
  auto up = [](size_t x) { return (x + 255) / 256 * 256; };
  size_t off = 0;
  L.x = off;
  off = up(off + size_t(bs) * MSA_BLOCK * s_pad * 2);
  L.rmax = off;
  off = up(off + size_t(bs) * MSA_BLOCK * 4);
  L.rsum = off;
  off = up(off + size_t(bs) * MSA_BLOCK * 8);
  L.vert = off;
  off = up(off + size_t(bs) * s * 4);
  L.slash = off;
  off = up(off + size_t(bs) * s * 4);
  L.total = off;
  return L;
}

size_t msa_vs_estimate_workspace_bytes(int64_t batch, int32_t n_slots, int64_t s,
                                       int32_t head_dim) {
  if (batch <= 0 || n_slots <= 0 || s <= 0 || head_dim <= 0) return 0;
  return vs_est_layout(batch, n_slots, s).total;
}

int msa_vs_estimate(const msa_tensor4* q, const msa_tensor4* k, const int32_t* slot_heads,
                    const int32_t* slot_vsize, const int32_t* slot_ssize, int32_t n_slots,
                    int32_t* v_idx, int32_t* v_cnt, int32_t v_stride, int32_t* s_idx,
                    int32_t* s_cnt, int32_t s_stride, void* workspace, size_t workspace_bytes,
                    msa_stream_t stream) {
  int st = check_qk(q, k);
  if (st != MSA_OK) return st;
  if (!vs_head_dim_ok(q->size[3])) return MSA_E_HEAD_DIM;
  if (!slot_heads || !slot_vsize || !slot_ssize || !v_idx || !v_cnt || !s_idx || !s_cnt)
    return MSA_E_NULL;
  const int64_t B = q->size[0], H = q->size[1], S = q->size[2];
  if (k->size[2] != S || S > kVsMaxSeq) return MSA_E_SEQ;
  if (n_slots < 1 || n_slots > kMaxHeads || B * n_slots > 65535) return MSA_E_SLOTS;
  if (v_stride < 1 || s_stride < 1) return MSA_E_SLOTS;
  for (int s = 0; s < n_slots; ++s) {
    if (slot_heads[s] < 0 || slot_heads[s] >= H) return MSA_E_HEADS;
    if (slot_vsize[s] < 1 || slot_vsize[s] > S || slot_vsize[s] > v_stride) return MSA_E_TOPK;
    if (slot_ssize[s] < 1 || slot_ssize[s] > S || slot_ssize[s] > s_stride) return MSA_E_TOPK;
  }
  const VsEstLayout L = vs_est_layout(B, n_slots, S);
  if (!workspace || workspace_bytes < L.total) return MSA_E_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return MSA_E_ALIGN;
  unsigned char* w = static_cast<unsigned char*>(workspace);
  VsEstParams p;
  memset(&p, 0, sizeof(p));
  p.q = q->data;
  p.k = k->data;
  p.q_sb = q->stride[0]; p.q_sh = q->stride[1]; p.q_ss = q->stride[2];
  p.k_sb = k->stride[0]; p.k_sh = k->stride[1]; p.k_ss = k->stride[2];
  p.batch = int(B);
  p.kv_group = int(H / k->size[1]);
  p.s = int(S);
  p.n_rows = int(std::min<int64_t>(MSA_BLOCK, S));
  p.n_slots = n_slots;
  p.s_pad = int(cdiv(S, MSA_BLOCK) * MSA_BLOCK);
  p.sqrt_d = float(std::sqrt(double(q->size[3])));
  p.x = reinterpret_cast<uint16_t*>(w + L.x);
  p.rmax = reinterpret_cast<float*>(w + L.rmax);
  p.rsum = reinterpret_cast<double*>(w + L.rsum);
  p.vert = reinterpret_cast<float*>(w + L.vert);
  p.slash = reinterpret_cast<float*>(w + L.slash);
  p.v_idx = v_idx;
  p.v_cnt = v_cnt;
  p.s_idx = s_idx;
  p.s_cnt = s_cnt;
  p.v_stride = v_stride;
  p.s_stride = s_stride;
  for (int s = 0; s < n_slots; ++s) {
    p.slot_heads[s] = int16_t(slot_heads[s]);
    p.slot_vsize[s] = slot_vsize[s];
    p.slot_ssize[s] = slot_ssize[s];
  }
  const hipError_t e =
      launch_vs_estimate(p, q->dtype, int(q->size[3]), reinterpret_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSA_OK : int(e);
}

size_t msa_vs_workspace_bytes(int64_t batch, int32_t n_slots, int64_t s_k, int32_t v_stride,
                              int32_t head_dim) {
  if (batch <= 0 || n_slots <= 0 || s_k <= 0 || v_stride <= 0 || head_dim <= 0) return 0;
  return vs_layout(batch, n_slots, s_k, v_stride, head_dim).total;
}

// Work model of one head for the XCD split: query block bq costs
// min(bq + 1, cap) + fixed, in key tiles (fixed covers the item set-up and
// the output merge).  The prefix sums have a closed form.
struct HeadWork {
  double cap, fixed;
  bool flat;  // every query block costs cap (no causal triangle)
};

static HeadWork head_work(const msa_head_desc& hd, int n_kb, int topk_max) {
  const double nb = double(n_kb);
  HeadWork w{nb, 2.0, hd.kind == MSA_KIND_FULL};
  if (hd.kind == MSA_KIND_STREAM) {
    w.cap = fmin(nb, double(hd.p2) / 64.0 + 2.0 + ceil(fmax(double(hd.p1), 0.0) / 64.0));
  } else if (hd.kind == MSA_KIND_BLOCK) {
    w.cap = fmin(nb, fmax(1.0, double(hd.p1 > 0 ? hd.p1 : topk_max)));
  } else if (hd.kind == MSA_KIND_VS) {
    // slash tiles grow with the slash count; vertical columns add gathered tiles
    w.cap = fmin(nb, 2.0 + double(hd.p2) / 16.0);
    w.fixed += double(hd.p1) / 128.0;
  }
  return w;
}

// cost of query blocks 0 .. m-1
static double prefix_cost(const HeadWork& w, double m) {
  const double k = w.cap;
  if (w.flat) return m * (k + w.fixed);
  const double tri = m <= k ? m * (m + 1) / 2 : k * (k + 1) / 2 + (m - k) * k;
  return tri + w.fixed * m;
}

// Items of one launch: the listed (batch, head) pairs, head-major, query
// blocks longest-first; the 8 XCDs (round-robin workgroup dispatch) take
// contiguous ranges of equal estimated cost, so each XCD's L2 serves few
// heads and a heavy head can be shared by two XCDs.
static void order_items(AttnParams& ap, const int* pairs, const HeadWork* work, int n) {
  const int nq = ap.n_qb;
  ap.n_hl = n;
  double head_tot[kMaxHeads], total = 0.0;
  for (int i = 0; i < n; ++i) {
    ap.head_order[i] = pairs[i];
    head_tot[i] = prefix_cost(work[i], nq);
    total += head_tot[i];
  }
  int prev = 0, h = 0;
  double before = 0.0;  // cost of the heads before h
  for (int x = 0; x < 8; ++x) {
    int cut = n * nq;
    if (x < 7) {
      const double target = total * (x + 1) / 8.0;
      while (h < n - 1 && before + head_tot[h] < target) before += head_tot[h++];
      const double need = target - before;
      int lo = 0, hi = nq;  // first r items (bq = nq-1 .. nq-r) of head h cost >= need
      while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (prefix_cost(work[h], nq) - prefix_cost(work[h], nq - mid) >= need) hi = mid;
        else lo = mid + 1;
      }
      cut = std::max(prev, h * nq + lo);
    }
    ap.xcd_start[x] = prev;
    ap.xcd_count[x] = cut - prev;
    prev = cut;
  }
}

// Puts the block_sparse entries of list[0..n) evenly between the others
// (stable within each group).  The XCDs take contiguous ranges of the item
// list, so this gives every XCD the same mix of L2-friendly band / dense
// heads and block heads, whose scattered tiles miss the L2 more.
static void interleave_kinds(int* list, int n, const msa_head_desc* heads, int H) {
  int blk[kMaxHeads], oth[kMaxHeads], nb = 0, no = 0;
  for (int i = 0; i < n; ++i) {
    if (heads[list[i] % H].kind == MSA_KIND_BLOCK) blk[nb++] = list[i];
    else oth[no++] = list[i];
  }
  int ib = 0, io = 0;
  for (int i = 0; i < n; ++i) {
    const bool take_b = ib < nb && (io >= no || int64_t(ib) * n <= int64_t(i) * nb);
    list[i] = take_b ? blk[ib++] : oth[io++];
  }
}

static int layer_attention_impl(const msa_tensor4* q, const msa_tensor4* k, const msa_tensor4* v,
                                const msa_tensor4* o, const msa_head_desc* heads, int32_t n_heads,
                                const int32_t* idx, const int32_t* cnt, int32_t idx_slots,
                                int32_t topk_max, const msa_vs_lists* vs, void* vs_workspace,
                                size_t vs_workspace_bytes, void* workspace,
                                size_t workspace_bytes, msa_stream_t stream, bool stage) {
  int st = check_qk(q, k);
  if (st != MSA_OK) return st;
  if (!v || !o || !v->data || !o->data || !heads) return MSA_E_NULL;
  for (int i = 0; i < 4; ++i) {
    if (v->size[i] != k->size[i]) return MSA_E_RANK;
    if (o->size[i] != q->size[i]) return MSA_E_RANK;
  }
  if (v->dtype != q->dtype) return MSA_E_DTYPE;
  if (o->dtype != q->dtype && o->dtype != MSA_DTYPE_FP32) return MSA_E_DTYPE;
  if (!aligned(v) || !aligned(o)) return MSA_E_ALIGN;
  const int64_t B = q->size[0], H = q->size[1], Hkv = k->size[1];
  const int64_t Sq = q->size[2], Sk = k->size[2];
  const int D = int(q->size[3]);
  if (n_heads != H || H > kMaxHeads) return MSA_E_HEADS;
  const int n_qb = int(cdiv(Sq, MSA_BLOCK));
  const int n_kb = int(cdiv(Sk, MSA_BLOCK));
  const int kv_group = int(H / Hkv);
  bool any_block = false;
  int n_vs = 0;
  for (int h = 0; h < n_heads; ++h) {
    const msa_head_desc& hd = heads[h];
    if (hd.kind == MSA_KIND_SKIP) continue;
    if (hd.kind != MSA_KIND_DENSE && hd.kind != MSA_KIND_STREAM && hd.kind != MSA_KIND_BLOCK &&
        hd.kind != MSA_KIND_VS && hd.kind != MSA_KIND_FULL)
      return MSA_E_HEADS;
    // S_q > S_k only without causal masking (no absolute row of the causal
    // kinds would exist for the first query rows)
    if (Sq > Sk && hd.kind != MSA_KIND_FULL) return MSA_E_SEQ;
    if (!(hd.scale > 0.0f) || !isfinite(hd.scale)) return MSA_E_HEADS;
    if (hd.kind == MSA_KIND_BLOCK) {
      any_block = true;
      if (hd.slot < 0 || hd.slot >= idx_slots) return MSA_E_SLOTS;
    }
    if (hd.kind == MSA_KIND_VS) ++n_vs;
  }
  if (any_block && (!idx || !cnt || topk_max < 1)) return MSA_E_SLOTS;
  VsLayout vl;
  int16_t slot_kvh[kMaxHeads];
  if (n_vs) {
    if (!vs_head_dim_ok(D)) return MSA_E_HEAD_DIM;
    if (!vs || !vs->v_idx || !vs->v_cnt || !vs->s_idx || !vs->s_cnt) return MSA_E_SLOTS;
    if (vs->n_slots < 1 || vs->n_slots > kMaxHeads || vs->v_stride < 1 ||
        vs->v_stride > kVsMaxSeq || vs->s_stride < 1)
      return MSA_E_SLOTS;
    if (Sq != Sk || Sk > kVsMaxSeq) return MSA_E_SEQ;
    if (B * H > kMaxHeads) return MSA_E_HEADS;
    for (int s = 0; s < vs->n_slots; ++s) slot_kvh[s] = -1;
    for (int h = 0; h < n_heads; ++h) {
      if (heads[h].kind != MSA_KIND_VS) continue;
      const int s = heads[h].slot;
      if (s < 0 || s >= vs->n_slots) return MSA_E_SLOTS;
      const int kvh = h / kv_group;
      if (slot_kvh[s] >= 0 && slot_kvh[s] != kvh) return MSA_E_SLOTS;
      slot_kvh[s] = int16_t(kvh);
    }
    for (int s = 0; s < vs->n_slots; ++s)
      if (slot_kvh[s] < 0) slot_kvh[s] = 0;  // unused slot: any kv head
    vl = vs_layout(B, vs->n_slots, Sk, vs->v_stride, D);
    if (!vs_workspace || vs_workspace_bytes < vl.total) return MSA_E_WORKSPACE;
    if ((reinterpret_cast<uintptr_t>(vs_workspace) & 255u) != 0) return MSA_E_ALIGN;
  }
  const size_t need = msa_attention_workspace_bytes(B, Hkv, Sk, D);
  if (!workspace || workspace_bytes < need) return MSA_E_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return MSA_E_ALIGN;
  if (int64_t(n_qb) * B * H > 0x7fffffffLL) return MSA_E_SEQ;
  if (B * Hkv > 65535) return MSA_E_HEADS;

  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  if (stage) {
    StageParams sp;
    st = stage_setup(k, v, workspace, workspace_bytes, sp);
    if (st == MSA_OK) st = stage_launch(sp, v->dtype, D, hs);
    if (st != MSA_OK) return st;
  }

  AttnParams ap;
  memset(&ap, 0, sizeof(ap));
  ap.q = q->data;
  ap.k = k->data;
  const AttnLayout AL = attn_layout(B, Hkv, Sk, D);
  ap.vt = ws_at<uint16_t>(workspace, AL.vt);
  ap.kt = ws_at<uint16_t>(workspace, AL.kt);
  ap.k_in_place = k_in_place(k) ? 1 : 0;
  int32_t* vexp = ws_at<int32_t>(workspace, AL.vexp);
  ap.vexp = vexp;
  ap.o = o->data;
  ap.q_sb = q->stride[0]; ap.q_sh = q->stride[1]; ap.q_ss = q->stride[2];
  ap.k_sb = k->stride[0]; ap.k_sh = k->stride[1]; ap.k_ss = k->stride[2];
  ap.o_sb = o->stride[0]; ap.o_sh = o->stride[1]; ap.o_ss = o->stride[2];
  ap.batch = int(B);
  ap.heads = int(H);
  ap.kv_group = kv_group;
  ap.s_q = int(Sq);
  ap.s_k = int(Sk);
  ap.n_qb = n_qb;
  ap.n_kb = n_kb;
  ap.s_pad = n_kb * MSA_BLOCK;
  ap.idx = idx;
  ap.cnt = cnt;
  ap.idx_slots = idx_slots;
  ap.topk_max = topk_max;
  ap.queue = queue_of(workspace, need);
  ap.wg_per_xcd = cus_per_xcd();
  const double log2e = 1.4426950408889634;
  for (int h = 0; h < n_heads; ++h) {
    const int kd = heads[h].kind;
    ap.hd[h].kind = kd;
    ap.hd[h].slot = kd == MSA_KIND_BLOCK || kd == MSA_KIND_VS ? heads[h].slot : 0;
    ap.hd[h].p1 = heads[h].p1;
    ap.hd[h].p2 = heads[h].p2;
    ap.hd[h].scale_log2 = float(double(heads[h].scale) * log2e);
  }

  const int BH = int(B * H);
  if (n_vs == 0) {
    if (BH <= kMaxHeads) {
      int pairs[kMaxHeads];
      HeadWork work[kMaxHeads];
      int n = 0;
      for (int i = 0; i < BH; ++i)
        if (heads[i % H].kind != MSA_KIND_SKIP) pairs[n++] = i;
      if (n == 0) return MSA_OK;
      interleave_kinds(pairs, n, heads, int(H));
      for (int i = 0; i < n; ++i) work[i] = head_work(heads[pairs[i] % H], n_kb, topk_max);
      order_items(ap, pairs, work, n);
    } else {
      ap.n_hl = 0;  // every pair, plain order
    }
    const hipError_t e = launch_attention(ap, q->dtype, o->dtype, D, hs);
    return e == hipSuccess ? MSA_OK : int(e);
  }

  // vertical_and_slash heads: tile lists, gathered vertical columns, launch
  unsigned char* vw = static_cast<unsigned char*>(vs_workspace);
  VsBuildParams bp;
  memset(&bp, 0, sizeof(bp));
  bp.v_idx = vs->v_idx;
  bp.v_cnt = vs->v_cnt;
  bp.s_idx = vs->s_idx;
  bp.s_cnt = vs->s_cnt;
  bp.lists = reinterpret_cast<uint32_t*>(vw + vl.lists);
  bp.cnt = reinterpret_cast<int32_t*>(vw + vl.cnt);
  bp.v_stride = vs->v_stride;
  bp.s_stride = vs->s_stride;
  bp.cap = vl.cap;
  bp.n_qb = n_qb;
  bp.n_kb = n_kb;
  bp.s_k = int(Sk);
  hipError_t e = launch_vs_build(bp, int(B) * vs->n_slots, hs);
  if (e != hipSuccess) return int(e);

  StageParams gp;
  memset(&gp, 0, sizeof(gp));
  gp.k = k->data;
  gp.v = v->data;
  gp.k_sb = k->stride[0]; gp.k_sh = k->stride[1]; gp.k_ss = k->stride[2];
  gp.v_sb = v->stride[0]; gp.v_sh = v->stride[1]; gp.v_ss = v->stride[2];
  gp.kt = reinterpret_cast<uint16_t*>(vw + vl.gk);
  gp.vt = reinterpret_cast<uint16_t*>(vw + vl.gv);
  gp.batch = int(B);
  gp.kv_heads = int(Hkv);
  gp.s_k = int(Sk);
  gp.s_pad = vl.nv_pad;
  gp.vexp = vexp;  // the heads' V exponents from the plain staging
  gp.rows = vs->v_idx;
  gp.rows_cnt = vs->v_cnt;
  gp.rows_stride = vs->v_stride;
  gp.n_slots = vs->n_slots;
  for (int s = 0; s < vs->n_slots; ++s) gp.slot_kvh[s] = slot_kvh[s];
  e = launch_stage(gp, q->dtype, D, hs);
  if (e != hipSuccess) return int(e);

  int vs_pairs[kMaxHeads], other[kMaxHeads];
  HeadWork vs_work[kMaxHeads], other_work[kMaxHeads];
  int n_v = 0, n_o = 0;
  for (int i = 0; i < BH; ++i) {
    const msa_head_desc& hd = heads[i % H];
    if (hd.kind == MSA_KIND_VS) {
      vs_pairs[n_v] = i;
      vs_work[n_v++] = head_work(hd, n_kb, topk_max);
    } else if (hd.kind != MSA_KIND_SKIP) {
      other[n_o++] = i;
    }
  }
  interleave_kinds(other, n_o, heads, int(H));
  for (int i = 0; i < n_o; ++i) other_work[i] = head_work(heads[other[i] % H], n_kb, topk_max);
  if (ap.k_in_place) {
    // the vertical_and_slash kernel reads staged K: stage the K the plain
    // staging left in place (V and its exponents are staged already)
    StageParams kp;
    st = stage_setup(k, v, workspace, workspace_bytes, kp);
    if (st != MSA_OK) return st;
    kp.stage_k = 2;
    e = launch_stage(kp, q->dtype, D, hs);
    if (e != hipSuccess) return int(e);
  }
  AttnParams vp = ap;
  vp.k_in_place = 0;
  vp.vs_lists = bp.lists;
  vp.vs_cnt = bp.cnt;
  vp.gkt = gp.kt;
  vp.gvt = gp.vt;
  vp.vs_slots = vs->n_slots;
  vp.vs_cap = vl.cap;
  vp.nv_pad = vl.nv_pad;
  order_items(vp, vs_pairs, vs_work, n_v);
  e = launch_attention_vs(vp, q->dtype, o->dtype, D, hs);
  if (e != hipSuccess) return int(e);
  if (n_o) {
    order_items(ap, other, other_work, n_o);
    e = launch_attention(ap, q->dtype, o->dtype, D, hs);
  }
  return e == hipSuccess ? MSA_OK : int(e);
}

int msa_layer_attention(const msa_tensor4* q, const msa_tensor4* k, const msa_tensor4* v,
                        const msa_tensor4* o, const msa_head_desc* heads, int32_t n_heads,
                        const int32_t* idx, const int32_t* cnt, int32_t idx_slots,
                        int32_t topk_max, void* workspace, size_t workspace_bytes,
                        msa_stream_t stream) {
  return layer_attention_impl(q, k, v, o, heads, n_heads, idx, cnt, idx_slots, topk_max,
                              nullptr, nullptr, 0, workspace, workspace_bytes, stream, true);
}

int msa_layer_attention_staged(const msa_tensor4* q, const msa_tensor4* k, const msa_tensor4* v,
                               const msa_tensor4* o, const msa_head_desc* heads, int32_t n_heads,
                               const int32_t* idx, const int32_t* cnt, int32_t idx_slots,
                               int32_t topk_max, void* workspace, size_t workspace_bytes,
                               msa_stream_t stream) {
  return layer_attention_impl(q, k, v, o, heads, n_heads, idx, cnt, idx_slots, topk_max,
                              nullptr, nullptr, 0, workspace, workspace_bytes, stream, false);
}

int msa_layer_attention_ex(const msa_tensor4* q, const msa_tensor4* k, const msa_tensor4* v,
                           const msa_tensor4* o, const msa_head_desc* heads, int32_t n_heads,
                           const int32_t* idx, const int32_t* cnt, int32_t idx_slots,
                           int32_t topk_max, const msa_vs_lists* vs, void* vs_workspace,
                           size_t vs_workspace_bytes, void* workspace, size_t workspace_bytes,
                           int32_t stage, msa_stream_t stream) {
  return layer_attention_impl(q, k, v, o, heads, n_heads, idx, cnt, idx_slots, topk_max, vs,
                              vs_workspace, vs_workspace_bytes, workspace, workspace_bytes,
                              stream, stage != 0);
}


// ---------------------------------------------------------------------------
// decode
// ---------------------------------------------------------------------------
// Key splits of one decode call: about 2048 workgroups in all, at least 64
// keys each.
static void decode_split(int64_t bh, int64_t s_k, int& n_split, int& chunk) {
  int64_t ns = (kDecodeMaxSplit + bh - 1) / bh;
  ns = std::max<int64_t>(1, std::min<int64_t>(ns, cdiv(s_k, 64)));
  int64_t ch = cdiv(s_k, ns);
  ch = cdiv(ch, 64) * 64;
  n_split = int(cdiv(s_k, ch));
  chunk = int(ch);
}

size_t msa_decode_workspace_bytes(int64_t batch, int64_t heads, int64_t s_k, int32_t head_dim) {
  if (batch <= 0 || heads <= 0 || s_k <= 0 || head_dim <= 0) return 0;
  int ns, ch;
  decode_split(batch * heads, s_k, ns, ch);
  const int64_t bytes = batch * heads * ns * (int64_t(head_dim) + 2) * 4;
  return size_t((bytes + 255) / 256 * 256);
}

int msa_decode_attention(const msa_tensor4* q, const msa_tensor4* k, const msa_tensor4* v,
                         const msa_tensor4* o, float scale, void* workspace,
                         size_t workspace_bytes, msa_stream_t stream) {
  int st = check_qk(q, k);
  if (st != MSA_OK) return st;
  if (!v || !o || !v->data || !o->data) return MSA_E_NULL;
  for (int i = 0; i < 4; ++i) {
    if (v->size[i] != k->size[i]) return MSA_E_RANK;
    if (o->size[i] != q->size[i]) return MSA_E_RANK;
  }
  if (q->size[2] != 1) return MSA_E_SEQ;
  if (v->dtype != q->dtype) return MSA_E_DTYPE;
  if (o->dtype != q->dtype && o->dtype != MSA_DTYPE_FP32) return MSA_E_DTYPE;
  if (!aligned(v) || !aligned(o)) return MSA_E_ALIGN;
  if (!(scale > 0.0f) || !isfinite(scale)) return MSA_E_HEADS;
  const int64_t B = q->size[0], H = q->size[1], Hkv = k->size[1], Sk = k->size[2];
  const int D = int(q->size[3]);
  // buffer descriptors cover one head's cache: < 2 GiB of rows
  if ((Sk + 64) * k->stride[2] * 2 >= (int64_t(1) << 31) ||
      (Sk + 64) * v->stride[2] * 2 >= (int64_t(1) << 31))
    return MSA_E_SEQ;
  if (B * H > 65535) return MSA_E_HEADS;
  const size_t need = msa_decode_workspace_bytes(B, H, Sk, D);
  if (!workspace || workspace_bytes < need) return MSA_E_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) return MSA_E_ALIGN;

  DecodeParams dp;
  memset(&dp, 0, sizeof(dp));
  dp.q = q->data; dp.k = k->data; dp.v = v->data; dp.o = o->data;
  dp.q_sb = q->stride[0]; dp.q_sh = q->stride[1];
  dp.k_sb = k->stride[0]; dp.k_sh = k->stride[1]; dp.k_ss = k->stride[2];
  dp.v_sb = v->stride[0]; dp.v_sh = v->stride[1]; dp.v_ss = v->stride[2];
  dp.o_sb = o->stride[0]; dp.o_sh = o->stride[1];
  dp.batch = int(B);
  dp.heads = int(H);
  dp.kv_group = int(H / Hkv);
  dp.s_k = int(Sk);
  decode_split(B * H, Sk, dp.n_split, dp.chunk);
  dp.scale_log2 = float(double(scale) * 1.4426950408889634);
  dp.part = static_cast<float*>(workspace);
  dp.ml = dp.part + B * H * dp.n_split * D;
  const hipError_t e = launch_decode(dp, q->dtype, o->dtype, D, reinterpret_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSA_OK : int(e);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// decode without allocation
// ---------------------------------------------------------------------------
// The split-K partials of msa_decode_attention_noalloc live in this array
// (each GPU holds its own copy until the process ends).  Host code must not
// pass `scratch` itself to a kernel: that name is a host-side stand-in.  Its
// device address is looked up once per device and kept in g_scratch.
static __device__ __align__(256) unsigned char scratch[MSA_DECODE_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// Device address of the current device's scratch; MSA_OK or a status.
int current_scratch(void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return int(e);
  if (dev < 0 || dev >= kMaxDevices) return int(hipErrorInvalidDevice);
  std::call_once(g_scratch_once[dev], [dev] {
    g_scratch_err[dev] = hipGetSymbolAddress(&g_scratch[dev], HIP_SYMBOL(scratch));
  });
  if (g_scratch_err[dev] != hipSuccess) return int(g_scratch_err[dev]);
  *out = g_scratch[dev];
  return MSA_OK;
}
}  // namespace

extern "C" {

int msa_decode_attention_noalloc(const msa_tensor4* q, const msa_tensor4* k,
                                 const msa_tensor4* v, const msa_tensor4* o, float scale,
                                 msa_stream_t stream) {
  // the same partials as msa_decode_attention; refuse what does not fit
  // before touching the device
  if (q && k && q->size[0] > 0 && q->size[1] > 0 && k->size[2] > 0 && q->size[3] > 0 &&
      q->size[3] <= 1024) {
    const size_t need = msa_decode_workspace_bytes(q->size[0], q->size[1], k->size[2],
                                                   int32_t(q->size[3]));
    if (need > size_t(MSA_DECODE_SCRATCH_BYTES)) return MSA_E_SCRATCH;
  }
  void* ws = nullptr;
  const int st = current_scratch(&ws);
  if (st != MSA_OK) return st;
  return msa_decode_attention(q, k, v, o, scale, ws, MSA_DECODE_SCRATCH_BYTES, stream);
}

int msa_rope_qk(const msa_tensor4* q, const msa_tensor4* k, const msa_tensor4* cos,
                const msa_tensor4* sin, const msa_tensor4* q_out, const msa_tensor4* k_out,
                msa_stream_t stream) {
  const msa_tensor4* all[6] = {q, k, cos, sin, q_out, k_out};
  for (const msa_tensor4* t : all) {
    if (!t || !t->data) return MSA_E_NULL;
    for (int i = 0; i < 4; ++i)
      if (t->size[i] <= 0) return MSA_E_RANK;
  }
  const int64_t B = q->size[0], H = q->size[1], S = q->size[2], D = q->size[3];
  const int64_t Hkv = k->size[1], rot = cos->size[3];
  if (k->size[0] != B || k->size[2] != S || k->size[3] != D) return MSA_E_RANK;
  for (int i = 0; i < 4; ++i)
    if (q_out->size[i] != q->size[i] || k_out->size[i] != k->size[i] ||
        sin->size[i] != cos->size[i])
      return MSA_E_RANK;
  if ((cos->size[0] != 1 && cos->size[0] != B) || cos->size[1] != 1 || cos->size[2] != S)
    return MSA_E_RANK;
  if (q->dtype != MSA_DTYPE_BF16 && q->dtype != MSA_DTYPE_FP16) return MSA_E_DTYPE;
  for (const msa_tensor4* t : all)
    if (t->dtype != q->dtype) return MSA_E_DTYPE;
  if (D % 8 != 0 || D > 512 || rot % 16 != 0 || rot > D || rot > kRopeMaxRot)
    return MSA_E_HEAD_DIM;
  for (const msa_tensor4* t : all)
    if (!aligned(t)) return MSA_E_ALIGN;
  const int64_t n_pair = rot / 16, n_pass = (D - rot) / 8;
  if (H + Hkv > 65535 || S > kMaxSeq || B > 65535)
    return MSA_E_SEQ;

  RopeParams rp;
  memset(&rp, 0, sizeof(rp));
  rp.q = q->data; rp.k = k->data; rp.cos = cos->data; rp.sin = sin->data;
  rp.qo = q_out->data; rp.ko = k_out->data;
  rp.q_sb = q->stride[0]; rp.q_sh = q->stride[1]; rp.q_ss = q->stride[2];
  rp.k_sb = k->stride[0]; rp.k_sh = k->stride[1]; rp.k_ss = k->stride[2];
  rp.qo_sb = q_out->stride[0]; rp.qo_sh = q_out->stride[1]; rp.qo_ss = q_out->stride[2];
  rp.ko_sb = k_out->stride[0]; rp.ko_sh = k_out->stride[1]; rp.ko_ss = k_out->stride[2];
  rp.c_sb = cos->size[0] == 1 ? 0 : cos->stride[0];
  rp.c_ss = cos->stride[2];
  rp.n_sb = sin->size[0] == 1 ? 0 : sin->stride[0];
  rp.n_ss = sin->stride[2];
  rp.batch = int(B); rp.heads = int(H); rp.kv_heads = int(Hkv); rp.s = int(S);
  rp.rot = int(rot); rp.half = int(rot / 2);
  rp.n_pair = int(n_pair); rp.n_pass = int(n_pass);
  const hipError_t e = launch_rope(rp, q->dtype, reinterpret_cast<hipStream_t>(stream));
  return e == hipSuccess ? MSA_OK : int(e);
}

}  // extern "C"
