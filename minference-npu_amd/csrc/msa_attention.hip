// Unified tile-list flash attention for one prefill layer (all heads, one grid).
//
// Work item = (head, 64-row query block).  Each item walks a list of 64-key
// tiles whose shape depends on the head kind:
//   dense        : every causal tile 0..diag              (backend_npu/attention.py:192-255)
//   full         : every key tile (dense, causal=False)   (backend_npu/attention.py:221-230)
//   stream_llm   : sink tiles, then the local band tiles  (ops/streaming_kernel_npu.py:94-146)
//   block_sparse : the estimator's block ids              (ops/block_sparse_kernel_npu.py:266-348,
//                                                          ops/tilelang_sparse_attention_h1.py:367-683)
// Token visibility (exact reference masks; row a is the absolute position
// i + S_k - S_q):
//   all kinds : j < S_k, and j <= a except for full heads
//   stream    : and (j > a - n_local or j < n_init)
// Rows with no visible key produce 0 (the reference's nan_to_num).
//
// CDNA4 mapping (one workgroup = 4 wave64 = one 64-row query block):
//   wave w owns all 64 query rows and the 16-key chunk [16w, 16w+16) of every
//   tile, with a private online-softmax state; the four chunk partials of a
//   row merge once at the end.  The main loop touches no LDS and has no
//   barrier: K and V operands go from L2 straight into registers.
//   S^T = K.Q^T on v_mfma_f32_16x16x32_{bf16,f16}: A = K chunk, B = Q
//   (registers for the whole item), one 16-row group per accumulator.  One
//   v_permlane16_swap per register pair turns two 16-row accumulators
//   (rounded to fp16) into the B operand of O^T = V^T.P^T on
//   v_mfma_f32_32x32x16_f16.  V is staged once per layer in exact operand
//   order as fp16, so every V operand is one contiguous 1 KB load; K is read
//   in place from the caller's rows (16 rows x 64 contiguous bytes per
//   operand load) unless its rows overlap or a head's rows span more than a
//   31-bit offset, or the launch is a vertical_and_slash one: then it is
//   staged in operand order too.
//   The exponentials are taken with each row's running max straight off
//   QK, biased so that a row's maximum has P = 2^7 (P, O and the row sums
//   all carry that factor, which cancels; it keeps small P out of fp16's
//   subnormal range); only when some P exceeds 2^15 (the row max grew by
//   more than 8 in log2 units) does a rare path recompute the half's scores,
//   reduce the row maxima over the four lanes of each row with permlane
//   swaps and rescale O.  Row sums accumulate per lane and reduce once at
//   the end.
//   Tiles that need no mask run first; boundary tiles (diagonal, band start,
//   partial sink, S_k end) run last with the elementwise mask.

#include <type_traits>

#include "msa_common.h"
#include "msa_kernels.h"
#include "msa_pool.h"

namespace msa {

#define INLINE __attribute__((always_inline))

constexpr int KIND_DENSE = 0;
constexpr int KIND_STREAM = 1;
constexpr int KIND_BLOCK = 2;
constexpr int KIND_VS = 3;
constexpr int KIND_FULL = 4;  // dense without the causal mask
constexpr int KIND_SKIP = 5;  // computed by another launch

// P = 2^(s*c - m) with m = (row max)*c - kPBias: a row's largest P is 2^7,
// and the rescale triggers above 2^kPSlackBits times that (2^15 < 65504, so
// every P handed to the fp16 PV product is finite).  The bias moves the
// fp16 subnormal range of P 7 bits further from the row maximum: a P of
// 2^-21 of the maximum still rounds with fp16's full relative precision.
constexpr float kPBias = 7.0f;
constexpr float kPCheck = 32768.0f;  // 2^(kPBias + 8)

// ---------------------------------------------------------------------------
// Per-layer staging of K and V into MFMA operand order, zero padded to
// s_pad = 64 * n_kb keys (chunk = 16 keys; 32-dim k-steps ks / blocks db):
//   Kop[B*Hkv][chunk][ks][lane 0..63][8], input dtype: lane l holds
//     K[16 chunk + (l & 15)][32 ks + 8 (l >> 4) + e]      (QK A operand, 16x16x32)
//   Vop[B*Hkv][chunk][db][lane 0..63][8], fp16: lane l holds
//     V[16 chunk + 8 (l >> 5) + e][32 db + (l & 31)]     (PV A operand, 32x32x16)
// so a wave reads every operand as one contiguous 1 KB.  Plane 1 stages K
// (a permutation of 16-byte granules; skipped where the attention kernel
// reads K in place), plane 0 stages V (a transpose through LDS, converted to
// fp16).  In gather mode the keys of a slot are
// the listed rows (the vertical columns of a vertical_and_slash head)
// instead of 0 .. s_k-1.
//
// V range: fp16 holds finite magnitudes up to 65504, bf16 far more.  A V
// tile is converted with saturation and reports its largest finite |V|
// (tmax); vscale_kernel then restages, times an exact power of two 2^-e, the
// V of any head whose maximum exceeds 65504, and the attention kernel
// multiplies that head's output by 2^e.  Inf and NaN are kept as they are.
// ---------------------------------------------------------------------------
template <int D>
struct StageShape {
  static constexpr int KCH = D / 8;   // 16-byte chunks per row
  static constexpr int NDB = D / 32;  // 32-dim operand blocks
  static constexpr int LP = D + 8;    // padded LDS row (halves)
};

// Source row of staged key j of head bk (-1: a zero key).
struct StageRows {
  const int32_t* rows;
  int rcnt, s_k;
  __device__ int operator()(int j) const {
    if (rows) return j < rcnt ? min(max(rows[j], 0), s_k - 1) : -1;
    return j < s_k ? j : -1;
  }
};

// V of 64 keys from j0 (staged row index) of head bk, times sc, into the
// operand layout; returns the largest finite |V| read (before scaling),
// reduced over the workgroup.  The caller must place a barrier between two
// calls that reuse `tile` / `red`.
template <typename T, int D>
__device__ float stage_v_tile(const StageParams& P, const uint16_t* src, const StageRows& src_row,
                              int64_t bk, int j0, float sc, uint16_t* tile, float* red) {
  using SS = StageShape<D>;
  constexpr int G = kBlock * SS::KCH / 256;  // 16-byte granules per thread
  static_assert(G * 256 == kBlock * SS::KCH, "whole granules per thread");
  // every load first, then the conversions
  u32x4 in[G];
  bool have[G];
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const int ci = threadIdx.x + 256 * u;
    const int r = ci / SS::KCH, c = ci - r * SS::KCH;
    const int j = src_row(j0 + r);
    have[u] = j >= 0;
    in[u] = have[u] ? load16(src + int64_t(j) * P.v_ss + c * 8) : zero_u32x4();
  }
  float vmax = 0.0f;
#pragma unroll
  for (int u = 0; u < G; ++u) {
    const int ci = threadIdx.x + 256 * u;
    const int r = ci / SS::KCH, c = ci - r * SS::KCH;
    u32x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float flo = T::to_float(uint16_t(in[u][e] & 0xffffu));
      const float fhi = T::to_float(uint16_t(in[u][e] >> 16));
      vmax = fmaxf(vmax, fmaxf(finite_abs(flo), finite_abs(fhi)));
      const _Float16 lo = to_f16_scaled(flo, sc);
      const _Float16 hi = to_f16_scaled(fhi, sc);
      out[e] = uint32_t(__builtin_bit_cast(uint16_t, lo)) |
               (uint32_t(__builtin_bit_cast(uint16_t, hi)) << 16);
    }
    store16(&tile[r * SS::LP + c * 8], out);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = vmax;
  __syncthreads();
  const int64_t dst0 = (bk * P.s_pad + j0) * D;
  u32x4 outv[SS::NDB];
#pragma unroll
  for (int u = 0; u < SS::NDB; ++u) {
    const int ci = threadIdx.x + 256 * u;
    const int l = ci & 63;
    const int cd = ci >> 6;  // chunk * NDB + db
    const int c = cd / SS::NDB, db = cd - c * SS::NDB;
    const int key0 = 16 * c + 8 * (l >> 5);
    const int d = 32 * db + (l & 31);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t lo = tile[(key0 + 2 * e) * SS::LP + d];
      const uint16_t hi = tile[(key0 + 2 * e + 1) * SS::LP + d];
      outv[u][e] = uint32_t(lo) | (uint32_t(hi) << 16);
    }
  }
#pragma unroll
  for (int u = 0; u < SS::NDB; ++u) store16(P.vt + dst0 + (threadIdx.x + 256 * u) * 8, outv[u]);
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Workgroup i of a launch: the first n_pool_wg run the block estimator's
// pooling pass (fused launch of msa_stage_kv_pool); then, in the dispatch
// order of a (tile, kv head, plane) grid, the V tiles of every kv head and
// then the K tiles (V only or K only as StageParams::stage_k says).
template <typename T, int D>
__global__ __launch_bounds__(256) void stage_kernel(StageParams P) {
  using SS = StageShape<D>;
  __shared__ __align__(16) uint16_t tile[kBlock * SS::LP];
  __shared__ float red[4];
  int wi = int(blockIdx.x);
  if (wi < P.n_pool_wg) {
    pool_workgroup<T, D>(P.pool, wi);
    return;
  }
  wi -= P.n_pool_wg;
  const int n_tiles = P.s_pad / kBlock;
  const int n_bk = P.batch * (P.rows ? P.n_slots : P.kv_heads);
  const int tile_i = wi % n_tiles;
  const int rest = wi / n_tiles;
  const int bk = rest % n_bk;  // b * kv_heads + kvh (gather mode: b * n_slots + slot)
  const int plane = P.stage_k == 2 ? 1 : rest / n_bk;  // 0: V, 1: K
  const int j0 = tile_i * kBlock;
  int b, kvh;
  StageRows src_row{nullptr, 0, P.s_k};
  if (P.rows) {
    b = bk / P.n_slots;
    kvh = P.slot_kvh[bk - b * P.n_slots];
    src_row.rows = P.rows + int64_t(bk) * P.rows_stride;
    src_row.rcnt = min(max(P.rows_cnt[bk], 0), P.rows_stride);
  } else {
    b = bk / P.kv_heads;
    kvh = bk - b * P.kv_heads;
  }
  // the tile's 4 chunks are 64*D consecutive halves starting at key j0
  const int64_t dst0 = (int64_t(bk) * P.s_pad + j0) * D;
  if (plane == 1) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(P.k) + b * P.k_sb + kvh * P.k_sh;
    // NDB granules per thread, every load before the stores
    u32x4 x[SS::NDB];
#pragma unroll
    for (int u = 0; u < SS::NDB; ++u) {
      const int gi = threadIdx.x + 256 * u;
      const int l = gi & 63;
      const int cks = gi >> 6;  // chunk * NDB + ks
      const int c = cks / SS::NDB, ks = cks - c * SS::NDB;
      // D > 128: the keys of each 32-key span in attn_wide_kernel's order
      // (8 (r / 4) + r % 4, then 8 (r / 4) + 4 + r % 4), so that each of its
      // K operands is one whole 16-key chunk
      const int q = 16 * c + (l & 15);
      const int kq = D > 128 ? 32 * (q >> 5) + 8 * ((q & 15) >> 2) + 4 * ((q >> 4) & 1) + (q & 3) : q;
      const int j = src_row(j0 + kq);
      x[u] = j >= 0 ? load16(src + int64_t(j) * P.k_ss + 32 * ks + 8 * (l >> 4)) : zero_u32x4();
    }
#pragma unroll
    for (int u = 0; u < SS::NDB; ++u) store16(P.kt + dst0 + (threadIdx.x + 256 * u) * 8, x[u]);
    return;
  }
  const uint16_t* src = reinterpret_cast<const uint16_t*>(P.v) + b * P.v_sb + kvh * P.v_sh;
  // gather mode uses the scale the head's plain staging chose
  const float sc = P.rows ? __builtin_amdgcn_ldexpf(1.0f, -P.vexp[b * P.kv_heads + kvh]) : 1.0f;
  const float m = stage_v_tile<T, D>(P, src, src_row, bk, j0, sc, tile, red);
  if (!P.rows && threadIdx.x == 0) P.tmax[int64_t(bk) * n_tiles + tile_i] = m;
}

// One workgroup per (batch, kv head): picks the head's V exponent from the
// tile maxima and, in the rare case it is not 0, restages the head's V.
template <typename T, int D>
__global__ __launch_bounds__(256) void vscale_kernel(StageParams P) {
  using SS = StageShape<D>;
  __shared__ __align__(16) uint16_t tile[kBlock * SS::LP];
  __shared__ float red[4];
  const int bk = blockIdx.x;
  const int n_kb = P.s_pad / kBlock;
  float m = 0.0f;
  for (int t = threadIdx.x; t < n_kb; t += 256) m = fmaxf(m, P.tmax[int64_t(bk) * n_kb + t]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  int e = 0;
  while (m * __builtin_amdgcn_ldexpf(1.0f, -e) > kF16Max) ++e;  // m < 2^128: e <= 113
  if (threadIdx.x == 0) P.vexp[bk] = e;
  if (e == 0) return;
  const int b = bk / P.kv_heads;
  const int kvh = bk - b * P.kv_heads;
  const uint16_t* src = reinterpret_cast<const uint16_t*>(P.v) + b * P.v_sb + kvh * P.v_sh;
  const StageRows src_row{nullptr, 0, P.s_k};
  const float sc = __builtin_amdgcn_ldexpf(1.0f, -e);
  for (int t = 0; t < n_kb; ++t) {
    stage_v_tile<T, D>(P, src, src_row, bk, t * kBlock, sc, tile, red);
    __syncthreads();  // tile and red are reused by the next tile
  }
}

template <typename T, int D>
static hipError_t launch_stage_t(const StageParams& p, hipStream_t st) {
  const int64_t n = p.n_pool_wg + int64_t(p.s_pad / kBlock) *
                                     (p.batch * (p.rows ? p.n_slots : p.kv_heads)) *
                                     (p.rows || p.stage_k == 1 ? 2 : 1);
  hipLaunchKernelGGL((stage_kernel<T, D>), dim3(uint32_t(n)), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_vscale_t(const StageParams& p, hipStream_t st) {
  hipLaunchKernelGGL((vscale_kernel<T, D>), dim3(p.batch * p.kv_heads), dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_stage(const StageParams& p, int dtype, int D, hipStream_t st) {
  if (dtype == Bf16::id) {
    if (D == 64) return launch_stage_t<Bf16, 64>(p, st);
    if (D == 96) return launch_stage_t<Bf16, 96>(p, st);
    if (D == 256) return launch_stage_t<Bf16, 256>(p, st);
    if (D == 512) return launch_stage_t<Bf16, 512>(p, st);
    return launch_stage_t<Bf16, 128>(p, st);
  }
  if (D == 64) return launch_stage_t<F16, 64>(p, st);
  if (D == 96) return launch_stage_t<F16, 96>(p, st);
  if (D == 256) return launch_stage_t<F16, 256>(p, st);
  if (D == 512) return launch_stage_t<F16, 512>(p, st);
  return launch_stage_t<F16, 128>(p, st);
}

hipError_t launch_vscale(const StageParams& p, int dtype, int D, hipStream_t st) {
  if (dtype == Bf16::id) {
    if (D == 64) return launch_vscale_t<Bf16, 64>(p, st);
    if (D == 96) return launch_vscale_t<Bf16, 96>(p, st);
    if (D == 256) return launch_vscale_t<Bf16, 256>(p, st);
    if (D == 512) return launch_vscale_t<Bf16, 512>(p, st);
    return launch_vscale_t<Bf16, 128>(p, st);
  }
  if (D == 64) return launch_vscale_t<F16, 64>(p, st);
  if (D == 96) return launch_vscale_t<F16, 96>(p, st);
  if (D == 256) return launch_vscale_t<F16, 256>(p, st);
  if (D == 512) return launch_vscale_t<F16, 512>(p, st);
  return launch_vscale_t<F16, 128>(p, st);
}

// ---------------------------------------------------------------------------
// attention
// ---------------------------------------------------------------------------
__device__ inline f32x16 mfma_pv(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Lane-row exchanges (a lane row = 16 consecutive lanes, R0..R3).
//   swap16(x, y): x <- [x.R0, y.R0, x.R2, y.R2], y <- [x.R1, y.R1, x.R3, y.R3]
//   swap32(x, y): x <- [x.R0, x.R1, y.R0, y.R1], y <- [x.R2, x.R3, y.R2, y.R3]
__device__ inline void swap16(uint32_t& x, uint32_t& y) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, y, false, false);
  x = r[0];
  y = r[1];
}
__device__ inline void swap16(float& x, float& y) {
  uint32_t a = __float_as_uint(x), b = __float_as_uint(y);
  swap16(a, b);
  x = __uint_as_float(a);
  y = __uint_as_float(b);
}
__device__ inline void swap32(float& x, float& y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  x = __uint_as_float(r[0]);
  y = __uint_as_float(r[1]);
}

// Row layouts of a wave's 64 query rows.  In the QK accumulator of row group
// g (rows 16g..16g+15) lane l holds 4 keys of row 16g + (l & 15); the 4 lane
// rows hold different keys of the same 16 rows ("group layout", one register
// per group).  A reduced row value lives one per lane in the "lane layout":
// lane l holds row 16 * rho(l >> 4) + (l & 15), rho = (0, 2, 1, 3).  The PV
// accumulator of row block rb holds row 32 rb + (l & 31) ("block layout").
struct RowSum {
  __device__ float operator()(float a, float b) const { return a + b; }
};

// group layout partials (4 groups) -> lane layout totals
template <typename Op>
__device__ inline float reduce_rows(float v0, float v1, float v2, float v3, Op op) {
  swap32(v0, v1);
  swap32(v2, v3);
  float a = op(v0, v1), b = op(v2, v3);
  swap16(a, b);
  return op(a, b);
}

// lane layout -> block layout of row blocks 0 and 1
__device__ inline void lanes_to_blocks(float u, float (&r)[2]) {
  float x = u, y = u;
  swap32(x, y);  // x = [g0, g2, g0, g2], y = [g1, g3, g1, g3]
  swap16(x, y);
  r[0] = x;
  r[1] = y;
}

// Tile sequence of one work item: up to five segments [lo_k, hi_k) laid end
// to end; positions before `mpos` hold tiles that need no mask, the rest the
// boundary tiles.  For block_sparse heads the segments index the id list,
// otherwise they are tile numbers.  Everything is wave-uniform (scalar
// registers) and position -> tile is branch-free, so the main loop is a plain
// counted loop.
struct TileSeq {
  int lo0, lo1, lo2, lo3, lo4;
  int c1, c2, c3, c4, total;  // start position of segments 1..4, end of segment 4
  int mpos;
  int n_kb;
  const int32_t* list;
  const int32_t* any;  // any readable int32 (the query tensor)

  __device__ void set(const int (&lo)[5], const int (&hi)[5], int nfull) {
    int c = 0;
    int cs[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) {
      cs[k] = c;
      c += max(hi[k] - lo[k], 0);
    }
    lo0 = lo[0]; lo1 = lo[1]; lo2 = lo[2]; lo3 = lo[3]; lo4 = lo[4];
    c1 = cs[1]; c2 = cs[2]; c3 = cs[3]; c4 = cs[4];
    total = c;
    mpos = nfull == 1 ? c1 : c2;
  }
  // Tile at position q, clamped into [0, n_kb) for memory safety; positions
  // past the end repeat the last tile (loads that are never consumed).  In
  // two halves, so that a caller can issue the scalar load a step before it
  // needs the tile: fetch (position -> index, and the list entry's load) and
  // finish (the tile from them).
  struct Pending {
    int v, i;
  };
  __device__ Pending fetch(int q) const {
    q = max(min(q, total - 1), 0);
    int i = lo4 + (q - c4);
    i = q < c4 ? lo3 + (q - c3) : i;
    i = q < c3 ? lo2 + (q - c2) : i;
    i = q < c2 ? lo1 + (q - c1) : i;
    i = q < c1 ? lo0 + q : i;
    // the load is unconditional (element 0 of `any` when there is no list)
    // so that no branch splits the caller's instruction stream
    return {load_uniform((list ? list : any) + (list ? i : 0)), i};
  }
  // PACKED: list entries are tile id << 16 | 16 key bits (the
  // vertical_and_slash lists)
  template <bool PACKED = false>
  __device__ int finish(Pending r) const {
    const int t = list ? (PACKED ? int(uint32_t(r.v) >> 16) : r.v) : r.i;
    return min(max(t, 0), n_kb - 1);
  }
  __device__ bool masked(int q) const { return q >= mpos; }
};

template <typename TO>
__device__ inline void store_out4(TO* dst, float a, float b, float c, float d);

template <>
__device__ inline void store_out4<float>(float* dst, float a, float b, float c, float d) {
  *reinterpret_cast<float4*>(dst) = make_float4(a, b, c, d);
}

template <typename T>
__device__ inline void store_out4_16(uint16_t* dst, float a, float b, float c, float d) {
  uint2 v;
  v.x = uint32_t(T::from_float(a)) | (uint32_t(T::from_float(b)) << 16);
  v.y = uint32_t(T::from_float(c)) | (uint32_t(T::from_float(d)) << 16);
  *reinterpret_cast<uint2*>(dst) = v;
}

template <int D>
struct AttnShape {
  static constexpr int NKS = D / 32;              // QK k-steps of 32 dims (= K loads per chunk)
  static constexpr int NDB = D / 32;              // PV output blocks of 32 dims (= V loads)
  static constexpr int CHUNK_BYTES = 16 * D * 2;  // one staged 16-key V chunk
  static constexpr int NO = NDB * 2 * 16;         // O accumulator floats per lane
  // merge area (floats): every wave's (m, l) of its rows, then per owner
  // wave v the three other waves' floats 4v .. 4v+3 of each O block
  static constexpr int ML = 4 * 64 * 4;
  static constexpr int MERGE = ML + 4 * 3 * (2 * NDB) * 64 * 4;
};

// Next item of the persistent attention grid: the home XCD's range first,
// then the others'; -1 when every range is empty.  One lane calls it.
__device__ inline int next_item(const AttnParams& P, int xcd) {
  for (int k = 0; k < 8; ++k) {
    const int y = (xcd + k) & 7;
    const int r = atomicAdd(&P.queue[y], 1);
    if (r < P.xcd_count[y]) return P.xcd_start[y] + r;
  }
  return -1;
}

__global__ void queue_reset_kernel(int* q) {
  if (threadIdx.x < 8) q[threadIdx.x] = 0;
}

// VS = false: stream_llm / block_sparse / dense heads; VS = true: the
// vertical_and_slash heads of a layer (tile lists from vs_build_kernel).
template <typename T, bool OUT_F32, int D, bool VS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D > 96 ? 1 : 2)))
void attn_kernel(AttnParams P) {
  using S = AttnShape<D>;
  constexpr int NKS = S::NKS;
  constexpr int NDB = S::NDB;
  __shared__ __align__(16) float lds[S::MERGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int lr = lane >> 4;  // lane row
  const int lc = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // keys 16w .. 16w+15 of every tile

  // ---- work items.  Workgroups are dispatched round-robin over the 8 XCDs
  // and each XCD takes a range of the head-major item list (query blocks
  // longest-first), so its L2 serves few heads at a time.
  //   vertical_and_slash (work known only after the tile-list build): the
  //   grid is persistent; a workgroup takes items of its XCD's range through
  //   that range's counter, then of the other XCDs' ranges once its own is
  //   empty, and exits when every range is empty.
  //   other kinds: workgroup i is item i / 8 of XCD i % 8's range (ranges
  //   cut by estimated cost); without a list, item i in plain order.  (A
  //   persistent grid over these items, resident workgroups taking items of
  //   their XCD's range with a static stride and requesting the next item's
  //   first tiles before the output merge, ran 12-15 % slower than one item
  //   per workgroup.)
  __shared__ int s_item;
  const int xcd = blockIdx.x & 7;

  // ---- state of the current work item (wave-uniform)
  int b = 0, h = 0, q0 = 0, a0 = 0, n_init = 0, n_local = 0, kind = KIND_DENSE;
  float c_log2 = 0.0f, vfac = 1.0f;
  TileSeq seq;
  __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.kt), short(0), 0, 0x00020000);
  __amdgpu_buffer_rsrc_t vrs = krs, gkrs = krs, gvrs = krs;
  __amdgpu_buffer_rsrc_t qrs = krs;  // the item's 64 query rows (rows past S_q out of range)
  int total = 0, mpos = 0, arow0 = 0, sink_hi = 0;
  bool is_full = false, is_stream = false;
  const int skm1 = P.s_k - 1;

  auto init_item = [&](const int hh, const int bq) INLINE {
    b = hh / P.heads;
    h = hh - b * P.heads;
    const int kvh = h / P.kv_group;
    const int hd_slot = P.hd[h].slot;
    kind = P.hd[h].kind;
    q0 = bq * kBlock;
    const int nrows = min(kBlock, P.s_q - q0);
    const int off = P.s_k - P.s_q;
    a0 = q0 + off;
    const int a1 = q0 + nrows - 1 + off;
    const int last_tile = min(a1 >> 6, P.n_kb - 1);
    n_init = P.hd[h].p1;
    n_local = P.hd[h].p2;
    // tile t needs no mask for the causal / S_k bounds iff t < F
    const int Fe = min(min((a0 + 1) >> 6, P.s_k >> 6), last_tile + 1);

    seq.n_kb = P.n_kb;
    seq.list = nullptr;
    seq.any = reinterpret_cast<const int32_t*>(P.q);
    if constexpr (VS) {
      // this wave's list: unmasked entries, then masked key tiles and
      // gathered vertical tiles (ids n_kb + g), each with its chunk's key bits
      const int64_t lrow = ((int64_t(b) * P.vs_slots + hd_slot) * P.n_qb + bq) * 4 + w;
      const int nf = load_uniform(P.vs_cnt + 2 * lrow);
      const int nt = load_uniform(P.vs_cnt + 2 * lrow + 1);
      seq.list = reinterpret_cast<const int32_t*>(P.vs_lists + lrow * P.vs_cap);
      seq.n_kb = P.n_kb + P.nv_pad / kBlock;
      seq.set({0, nf, 0, 0, 0}, {nf, nt, 0, 0, 0}, 1);
    } else if (kind == KIND_BLOCK) {
      // canonical list: ascending causal ids, so the boundary ids come last
      const int64_t base = (int64_t(b) * P.idx_slots + hd_slot) * P.n_qb + bq;
      const int cnt = max(0, min(load_uniform(P.cnt + base), P.topk_max));
      const int32_t* list = P.idx + base * P.topk_max;
      int nf = cnt;
      while (nf > 0 && load_uniform(list + nf - 1) >= Fe) --nf;
      seq.list = list;
      seq.set({0, nf, 0, 0, 0}, {nf, cnt, 0, 0, 0}, 1);
    } else if (kind == KIND_STREAM) {
      const int lo = min(max(a0 - n_local + 1, 0) >> 6, last_tile + 1);
      const int nsink = min((min(max(n_init, 0), P.s_k) + 63) >> 6, lo);
      const int sf = max(0, min(nsink, min(n_init >> 6, Fe)));  // sink tiles below n_init
      int bf0 = a1 - n_local + 1;                                 // band tiles in every row's band
      bf0 = bf0 <= 0 ? 0 : (bf0 + 63) >> 6;
      bf0 = min(max(bf0, lo), last_tile + 1);
      const int fb_hi = max(bf0, Fe);
      // full sink, full band | partial sink, band tiles cut by the window
      // start, diagonal / S_k boundary
      seq.set({0, bf0, sf, lo, fb_hi}, {sf, fb_hi, nsink, bf0, last_tile + 1}, 2);
    } else if (kind == KIND_FULL) {
      const int ff = P.s_k >> 6;  // tiles whose keys are all below S_k
      seq.set({0, ff, 0, 0, 0}, {ff, P.n_kb, 0, 0, 0}, 1);
    } else {
      seq.set({0, Fe, 0, 0, 0}, {Fe, last_tile + 1, 0, 0, 0}, 1);
    }
    total = seq.total;
    mpos = min(seq.mpos, total);

    const int64_t bk = int64_t(b) * (P.heads / P.kv_group) + kvh;
    // staged V is V * 2^-vexp (stage_kernel); the output takes the 2^vexp back
    vfac = __builtin_amdgcn_ldexpf(1.0f, load_uniform(P.vexp + bk));
    if (!VS && P.k_in_place) {
      // the head's own K rows; the record count ends at the last row's last
      // element, so rows past S_k (and dropped loads) read zeros
      krs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(P.k) + b * P.k_sb +
                                int64_t(kvh) * P.k_sh),
          short(0), int(((P.s_k - 1) * P.k_ss + D) * 2), 0x00020000);
    } else {
      krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.kt + bk * P.s_pad * D),
                                              short(0), P.s_pad * D * 2, 0x00020000);
    }
    vrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.vt + bk * P.s_pad * D),
                                            short(0), P.s_pad * D * 2, 0x00020000);
    // gathered vertical operands of a vertical_and_slash slot (tiles n_kb + g)
    if constexpr (VS) {
      const int64_t gb = (int64_t(b) * P.vs_slots + hd_slot) * P.nv_pad * D;
      gkrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.gkt + gb), short(0),
                                               P.nv_pad * D * 2, 0x00020000);
      gvrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(P.gvt + gb), short(0),
                                               P.nv_pad * D * 2, 0x00020000);
    }
    // the item's rows of Q: row q0 + r at byte r * q_ss * 2.  The record
    // count ends at the last row's last element, so every load of a row past
    // S_q either lies beyond it (zeros) or reads memory of the view (a row
    // stride below D: overlapping or repeated rows); rows past S_q feed only
    // their own, never stored, outputs.
    qrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(P.q) + b * P.q_sb +
                              int64_t(h) * P.q_sh + int64_t(q0) * P.q_ss),
        short(0), int(((nrows - 1) * P.q_ss + D) * 2), 0x00020000);
    c_log2 = P.hd[h].scale_log2;
    arow0 = a0 + lc;  // absolute position of this lane's row in group 0
    is_full = kind == KIND_FULL;
    is_stream = kind == KIND_STREAM;
    sink_hi = is_stream ? n_init : 0;
  };

  // ---- Q as the B operand: lane (lc, lr) of group g, k-step ks holds
  // Q[q0 + 16g + lc][32ks + 8lr .. +7]; rows past S_q are zero
  u32x4 qb[4][NKS];
  auto load_q = [&]() INLINE {
    if constexpr (VS) {
      // vertical_and_slash: plain loads of row min(row, S_q - 1), rows past
      // S_q zeroed after the load (fewer registers in this variant)
      const uint16_t* qbase =
          reinterpret_cast<const uint16_t*>(P.q) + b * P.q_sb + int64_t(h) * P.q_sh;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int row = q0 + 16 * g + lc;
        const int64_t roff = int64_t(min(row, P.s_q - 1)) * P.q_ss;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qb[g][ks] = load16(qbase + roff + 32 * ks + 8 * lr);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
          qb[g][ks] = q0 + 16 * g + lc < P.s_q ? qb[g][ks] : zero_u32x4();
      return;
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t roff = uint32_t((16 * g + lc) * P.q_ss * 2 + 16 * lr);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        qb[g][ks] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(qrs, roff, 64 * ks, 0));
    }
  };

  // K and V chunk operands of tile t: wave w reads chunk c = 4t + w.  Staged
  // operands: each MFMA operand is one contiguous 1 KB (lane l: 16 bytes).
  // K in place (not in vertical_and_slash launches, whose K is staged): lane
  // (lc, lr) of k-step ks reads K row 16c + lc at elements 32 ks + 8 lr ..
  // +7; the row offset sits in the lane's VGPR, so a row past S_k is out of
  // the buffer's range on its own.  drop: the position lies past the item's
  // last tile; the lane offset is then out of the buffer's range, so the
  // load returns zeros without a memory access (the loop's instruction
  // stream stays the same).
  const uint32_t lane_off = 16u * lane;
  const bool k_in_place = !VS && P.k_in_place;
  const uint32_t k_row_bytes = uint32_t(P.k_ss) * 2u;
  const uint32_t k_lane = k_in_place ? uint32_t(lc) * k_row_bytes + 16u * lr : lane_off;
  const uint32_t k_cv = k_in_place ? 16u * k_row_bytes : 0u;  // VGPR bytes per chunk
  const int k_cs = k_in_place ? 0 : S::CHUNK_BYTES;          // SGPR bytes per chunk
  const int k_kss = k_in_place ? 64 : 1024;                  // bytes per k-step
  auto load_k = [&](int t, u32x4 (&kr)[NKS], bool drop) INLINE {
    if constexpr (VS) {
      const bool gat = t >= P.n_kb;
      const __amdgpu_buffer_rsrc_t rs = gat ? gkrs : krs;
      t = gat ? t - P.n_kb : t;
      const int soff = (4 * t + w) * S::CHUNK_BYTES;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        kr[ks] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane_off, soff + 1024 * ks, 0));
    } else {
      const int c = 4 * t + w;
      const uint32_t vo = (k_lane + uint32_t(c) * k_cv) | (drop ? 0x80000000u : 0u);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        kr[ks] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, vo, c * k_cs + k_kss * ks, 0));
    }
  };
  auto load_v = [&](int t, u32x4 (&vr)[NDB], bool drop) INLINE {
    __amdgpu_buffer_rsrc_t rs = vrs;
    if constexpr (VS) {
      const bool gat = t >= P.n_kb;
      rs = gat ? gvrs : vrs;
      t = gat ? t - P.n_kb : t;
    }
    const int soff = (4 * t + w) * S::CHUNK_BYTES;
    const uint32_t vo = lane_off | (drop ? 0x80000000u : 0u);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      vr[db] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, vo, soff + 1024 * db, 0));
  };

  f32x16 o[NDB][2];
  // Running (biased) max per row in scaled log2 units, group layout (each
  // group's value in all 4 lane rows).  It only moves when some P would
  // exceed 2^15, so the O rescale is rare.
  float m_g[4];
  float l_g[4];  // per-lane partial row sums, group layout
  auto reset_acc = [&]() INLINE {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][rb][i] = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      m_g[g] = -1e30f;
      l_g[g] = 0.0f;
    }
  };

  // A step works on two 32-row halves h (groups 2h, 2h+1 = PV row block h) so
  // that the softmax of one half overlaps the MFMAs of the other.
  auto qk_half = [&](const u32x4 (&kr)[NKS], int hf, f32x4 (&s)[2]) INLINE {
    s[0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    s[1] = s[0];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) s[gg] = mfma_qk<T>(kr[ks], qb[2 * hf + gg][ks], s[gg]);
  };
  // visible iff j <= key_hi and (j >= band_lo or j < sink_hi); for a
  // vertical_and_slash tile: iff the key's bit is set in the wave's chunk
  // mask mk (16 bits) and (gathered tile, all keys in every row's past, or
  // j <= key_hi)
  auto mask_half = [&](f32x4 (&s)[2], int hf, int t, uint32_t mk) INLINE {
    const int jb = t * kBlock + 16 * w + 4 * lr;
    uint32_t bits = 0xfu;
    bool past = false;
    if constexpr (VS) {
      bits = (mk >> (4 * lr)) & 0xfu;
      past = t >= P.n_kb;
      // every key of a gathered tile or of a tile before the first row's
      // tile lies in every row's past: visibility is the key's bit, the same
      // for all rows of a lane (wave-uniform branch)
      if (past || t * kBlock + kBlock - 1 < a0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool on = (bits >> i) & 1u;
#pragma unroll
          for (int gg = 0; gg < 2; ++gg) s[gg][i] = on ? s[gg][i] : -__builtin_inff();
        }
        return;
      }
    }
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      const int ar = arow0 + 16 * (2 * hf + gg);
      const int key_hi = is_full ? skm1 : min(ar, skm1);
      const int band_lo = is_stream ? ar - n_local + 1 : 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = jb + i;
        bool vis;
        if constexpr (VS) {
          vis = ((bits >> i) & 1u) && (past || j <= key_hi);
        } else {
          vis = (j <= key_hi) & ((j >= band_lo) | (j < sink_hi));
        }
        s[gg][i] = vis ? s[gg][i] : -__builtin_inff();
      }
    }
  };
  // P = 2^(s*c - m) in place, with the current running max, and ps[gg] =
  // the lane's sum of its four P of group gg (its share of the row sum).
  // Returns true when some sum exceeds 2^15; every P is at most its sum
  // (P >= 0), so otherwise no P is large enough to need a rescale.
  auto exp_half = [&](f32x4 (&s)[2], int hf, float (&ps)[2]) INLINE -> bool {
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        s[gg][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[gg][i], c_log2, -m_g[2 * hf + gg]));
      ps[gg] = (s[gg][0] + s[gg][1]) + (s[gg][2] + s[gg][3]);
    }
    return __ballot(fmaxf(ps[0], ps[1]) > kPCheck) != 0;
  };
  // Rare path: recompute the half's scores, raise the running max to the
  // row max, rescale the half's O and row sums, and redo the exponentials.
  auto rescale_half = [&](const u32x4 (&kr)[NKS], f32x4 (&s)[2], float (&ps)[2], int hf, int t,
                          uint32_t mk, bool mt) INLINE {
    qk_half(kr, hf, s);
    if (mt) mask_half(s, hf, t, mk);
    float m0 = fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3]));
    float m1 = fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3]));
    swap32(m0, m1);  // lane rows (R0, R2) and (R1, R3) of each group
    float a = fmaxf(m0, m1), bb = a;
    swap16(a, bb);
    float g0 = fmaxf(a, bb), g1 = g0;  // [group 2h, 2h, 2h+1, 2h+1] by lane row
    swap32(g0, g1);                    // g0: group 2h in every lane row, g1: group 2h+1
    const float n0 = fmaxf(m_g[2 * hf], g0 * c_log2 - kPBias);
    const float n1 = fmaxf(m_g[2 * hf + 1], g1 * c_log2 - kPBias);
    const float al0 = __builtin_amdgcn_exp2f(m_g[2 * hf] - n0);
    const float al1 = __builtin_amdgcn_exp2f(m_g[2 * hf + 1] - n1);
    m_g[2 * hf] = n0;
    m_g[2 * hf + 1] = n1;
    l_g[2 * hf] *= al0;
    l_g[2 * hf + 1] *= al1;
    const float ab = (lr & 1) ? al1 : al0;  // block layout: lane rows 1, 3 hold group 2h+1
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[db][hf][i] *= ab;
    exp_half(s, hf, ps);
  };
  // Row sums take the fp32 P (the half's ps), P rounded to fp16 goes to
  // PV: groups 2h, 2h+1 -> B operand of row block h (keys 8(l>>5) .. +7 of
  // row 32h + (l&31)) with one lane-row swap per register pair.
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  auto pv_half = [&](const f32x4 (&s)[2], const float (&ps)[2], int hf,
                     const u32x4 (&vr)[NDB]) INLINE {
    uint32_t pk[2][2];
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      pk[gg][0] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{s[gg][0], s[gg][1]}, h2));
      pk[gg][1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{s[gg][2], s[gg][3]}, h2));
      l_g[2 * hf + gg] += ps[gg];
    }
    uint32_t x0 = pk[0][0], y0 = pk[1][0], x1 = pk[0][1], y1 = pk[1][1];
    swap16(x0, y0);
    swap16(x1, y1);
    const u32x4 pb = u32x4{x0, x1, y0, y1};
    // O^T[d][row] += V^T[d][key] . P^T[key][row]
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db][hf] = mfma_pv(vr[db], pb, o[db][hf]);
  };

  // Pipeline over positions p: two register sets alternate (A: even p, B:
  // odd p).  The K operands of position p+2 are requested as soon as QK of p
  // has consumed the set, the V operands once PV has.  Loads are issued
  // unconditionally (past the item's end they are dropped), so every path
  // through the loop has the same loads in flight and the waits stay exact.
  // The tile number of p+3 is looked up one step before its loads.  Tiles
  // that need no mask and boundary tiles run as two separate loops (the mask
  // is a compile-time switch, so no branch splits a step's instruction
  // stream); each loop runs whole (A, B) pairs, with a single step before or
  // after it when its range starts or ends on the other set.
  u32x4 kA[NKS], vA[NDB], kB[NKS], vB[NDB];
  // key masks of vertical_and_slash tiles come in the list entries with
  // their tile numbers
  auto mask_of = [&](TileSeq::Pending r) INLINE -> uint32_t {
    if constexpr (VS) return uint32_t(r.v) & 0xffffu;
    return 0u;
  };
  int tA = 0, tB = 0;
  TileSeq::Pending pn{0, 0};  // lookup of the position two ahead, issued a step early
  uint32_t mA = 0, mB = 0;
  // the first two positions' operands of the item (and the third's tile)
  auto start_tiles = [&]() INLINE {
    const TileSeq::Pending p0 = seq.fetch(0), p1 = seq.fetch(1);
    tA = seq.template finish<VS>(p0);
    tB = seq.template finish<VS>(p1);
    mA = mask_of(p0);
    mB = mask_of(p1);
    load_k(tA, kA, !VS && total < 1);
    load_v(tA, vA, !VS && total < 1);
    load_k(tB, kB, !VS && total < 2);
    load_v(tB, vB, !VS && total < 2);
    pn = seq.fetch(2);
  };
  // one step: QK of both halves; half 0's softmax under half 1's QK, half
  // 1's softmax under half 0's PV; K is reloaded once the rare path can no
  // longer need it
  auto step = [&](auto masked, u32x4 (&kr)[NKS], u32x4 (&vr)[NDB], int& tcur, uint32_t& mcur,
                  int p) INLINE {
    constexpr bool MT = decltype(masked)::value;
    // the tile of position p + 2 from the lookup issued in the previous step
    // (its scalar load has had a step to arrive), then position p + 3's
    // lookup.  (A scheduling barrier pinning that load here cost 1.5 %.)
    const int tn = seq.template finish<VS>(pn);
    const uint32_t mnext = mask_of(pn);
    pn = seq.fetch(p + 3);
    // (vertical_and_slash items walk long lists: the per-step test costs
    // more there than the two loads it saves per item)
    const bool drop = !VS && p + 2 >= total;
    f32x4 sa[2], sb[2];
    float pa[2], pb[2];
    qk_half(kr, 0, sa);
    qk_half(kr, 1, sb);
    if constexpr (MT) mask_half(sa, 0, tcur, mcur);
    if (exp_half(sa, 0, pa)) rescale_half(kr, sa, pa, 0, tcur, mcur, MT);
    pv_half(sa, pa, 0, vr);
    if constexpr (MT) mask_half(sb, 1, tcur, mcur);
    if (exp_half(sb, 1, pb)) rescale_half(kr, sb, pb, 1, tcur, mcur, MT);
    load_k(tn, kr, drop);
    pv_half(sb, pb, 1, vr);
    load_v(tn, vr, drop);
    tcur = tn;
    mcur = mnext;
  };
  auto run = [&](auto masked, int p0, int p1) INLINE {
    int p = p0;
    if ((p & 1) && p < p1) step(masked, kB, vB, tB, mB, p++);
    for (; p + 1 < p1; p += 2) {
      step(masked, kA, vA, tA, mA, p);
      step(masked, kB, vB, tB, mB, p + 1);
    }
    if (p < p1) step(masked, kA, vA, tA, mA, p);
  };
  auto body = [&]() INLINE {
    run(std::integral_constant<bool, false>(), 0, mpos);
    run(std::integral_constant<bool, true>(), mpos, total);
  };

  // ---- merge the four chunk partials of each row and write the item's rows
  // (batch ib, head ih, first row iq0; iv = 2^vexp of its head).  Wave v
  // owns floats 4v .. 4v+3 of every O block (output columns 32 db + 8 v ..
  // +7): every wave puts its (m, l) and the other owners' floats in LDS,
  // then combines and stores its own columns.  Block layout: lane rows 1, 3
  // hold group 2rb+1, chosen by an exact blend (the maxima are finite)
  // rather than a select, which the compiler turns into a lane-indexed load
  // from a private copy of m_g.
  auto merge_store = [&](const int ib, const int ih, const int iq0, const float iv) INLINE {
    float m_b[2], l_b[2];
    const float odd = float(lr & 1);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
      m_b[rb] = __builtin_fmaf(odd, m_g[2 * rb + 1], (1.0f - odd) * m_g[2 * rb]);
    lanes_to_blocks(reduce_rows(l_g[0], l_g[1], l_g[2], l_g[3], RowSum()), l_b);
    float4* ml = reinterpret_cast<float4*>(lds);
    // part[((v * 3 + k) * 2 NDB + db * 2 + rb) * 64 + lane]: floats 4v .. 4v+3
    // of o[db][rb] of wave c (k = c < v ? c : c - 1) for owner v
    float4* part = reinterpret_cast<float4*>(lds + S::ML);
    ml[w * 64 + lane] = make_float4(m_b[0], m_b[1], l_b[0], l_b[1]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if (v == w) continue;
      const int k = w < v ? w : w - 1;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          part[((v * 3 + k) * 2 * NDB + db * 2 + rb) * 64 + lane] =
              make_float4(o[db][rb][4 * v], o[db][rb][4 * v + 1], o[db][rb][4 * v + 2],
                          o[db][rb][4 * v + 3]);
    }
    __syncthreads();
    float4 mlc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) mlc[c] = ml[c * 64 + lane];
    auto combine = [&](auto wc) INLINE {
      constexpr int W = decltype(wc)::value;
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        float mw[4], lw[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          mw[c] = rb ? mlc[c].y : mlc[c].x;
          lw[c] = rb ? mlc[c].w : mlc[c].z;
        }
        const float mt = fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3]));
        float f[4];
        float lt = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          f[c] = __builtin_amdgcn_exp2f(mw[c] - mt);
          lt += lw[c] * f[c];
        }
        const float inv = lt > 0.0f ? iv / lt : 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) f[c] *= inv;

        const int row = iq0 + 32 * rb + (lane & 31);
        if (row < P.s_q) {
          const int64_t obase = ib * P.o_sb + int64_t(ih) * P.o_sh + int64_t(row) * P.o_ss;
#pragma unroll
          for (int db = 0; db < NDB; ++db) {
            float4 pc[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              if (c == W) {
                pc[c] = make_float4(o[db][rb][4 * W], o[db][rb][4 * W + 1], o[db][rb][4 * W + 2],
                                    o[db][rb][4 * W + 3]);
              } else {
                const int k = c < W ? c : c - 1;
                pc[c] = part[((W * 3 + k) * 2 * NDB + db * 2 + rb) * 64 + lane];
              }
            }
            // the four waves' terms added in wave order, one rounding each
            float v4[4] = {pc[0].x * f[0], pc[0].y * f[0], pc[0].z * f[0], pc[0].w * f[0]};
#pragma unroll
            for (int c = 1; c < 4; ++c) {
              v4[0] = __builtin_fmaf(pc[c].x, f[c], v4[0]);
              v4[1] = __builtin_fmaf(pc[c].y, f[c], v4[1]);
              v4[2] = __builtin_fmaf(pc[c].z, f[c], v4[2]);
              v4[3] = __builtin_fmaf(pc[c].w, f[c], v4[3]);
            }
            const int d = 32 * db + 8 * W + 4 * (lane >> 5);
            if constexpr (OUT_F32) {
              store_out4<float>(reinterpret_cast<float*>(P.o) + obase + d, v4[0], v4[1], v4[2],
                                v4[3]);
            } else {
              store_out4_16<T>(reinterpret_cast<uint16_t*>(P.o) + obase + d, v4[0], v4[1],
                               v4[2], v4[3]);
            }
          }
        }
      }
    };
    if (w == 0) combine(std::integral_constant<int, 0>());
    else if (w == 1) combine(std::integral_constant<int, 1>());
    else if (w == 2) combine(std::integral_constant<int, 2>());
    else combine(std::integral_constant<int, 3>());
  };

  if constexpr (VS) {
    for (;;) {
      if (tid == 0) s_item = next_item(P, xcd);
      __syncthreads();
      const int g = __builtin_amdgcn_readfirstlane(s_item);
      __syncthreads();
      if (g < 0) break;
      const int hl = g / P.n_qb;
      init_item(int(P.head_order[hl]), P.n_qb - 1 - (g - hl * P.n_qb));
      load_q();
      reset_acc();
      start_tiles();
      body();
      merge_store(b, h, q0, vfac);
    }
  } else {
    int hh, bq;
    if (P.n_hl) {
      const int r = int(blockIdx.x) >> 3;
      if (r >= P.xcd_count[xcd]) return;
      const int g = P.xcd_start[xcd] + r;
      const int hl = g / P.n_qb;
      hh = int(P.head_order[hl]);
      bq = P.n_qb - 1 - (g - hl * P.n_qb);
    } else {
      // plain order: every (batch, head) pair; the host lists no item of a
      // skipped head in the other modes
      const int BH = P.batch * P.heads;
      hh = int(blockIdx.x) % BH;
      if (P.hd[hh % P.heads].kind == KIND_SKIP) return;
      bq = P.n_qb - 1 - int(blockIdx.x) / BH;
    }
    init_item(hh, bq);
    load_q();
    reset_acc();
    start_tiles();
    body();
    merge_store(b, h, q0, vfac);
  }
}

// ---------------------------------------------------------------------------
// Head dims 256 and 512 (the ops zero-pad head dims 129..511 to them).  The
// same work items and tile walk as attn_kernel; the O of 64 rows x D does
// not fit one wave, so wave w owns the 16 query rows 16w .. 16w+15 and walks
// every key of the item's tiles itself (no merge).  Each 32-key span of a
// tile gives two 16x16x32 QK accumulators whose rows are the keys
//   A: 8 (r / 4) + (r % 4),   B: 8 (r / 4) + 4 + (r % 4)   (r = accumulator row)
// (the staging writes K of this head dim in that key order, so each QK
// operand is one contiguous staged 16-key chunk), so lane l holds keys
// 8 (l / 16) .. +7 of its query row l % 16: rounded to fp16 they are the B
// operand of the 16x16x32 PV product as they stand.  V comes from the staged
// 32x32x16 operand layout, one 16-byte granule per lane.  The row max is
// exact per tile (O rescaled when it grows), P biased to 2^kPBias like
// attn_kernel; fully masked rows give 0.  At D = 512 one wave per SIMD (the
// O accumulators, a K chunk and a V span take about 500 registers).
template <typename T, bool OUT_F32, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D > 256 ? 1 : 2)))
void attn_wide_kernel(AttnParams P) {
  static_assert(D == 256 || D == 512, "wide head dims");
  constexpr int NKS = D / 32;  // QK k-steps
  constexpr int NDO = D / 16;  // PV output blocks of 16 dims
  constexpr int NDB = D / 32;  // staged V blocks of 32 dims per 16-key chunk
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int lr = lane >> 4;
  const int lc = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int xcd = blockIdx.x & 7;
  int hh, bq;
  if (P.n_hl) {
    const int r = int(blockIdx.x) >> 3;
    if (r >= P.xcd_count[xcd]) return;
    const int g = P.xcd_start[xcd] + r;
    const int hl = g / P.n_qb;
    hh = int(P.head_order[hl]);
    bq = P.n_qb - 1 - (g - hl * P.n_qb);
  } else {
    const int BH = P.batch * P.heads;
    hh = int(blockIdx.x) % BH;
    if (P.hd[hh % P.heads].kind == KIND_SKIP) return;
    bq = P.n_qb - 1 - int(blockIdx.x) / BH;
  }
  const int b = hh / P.heads;
  const int h = hh - b * P.heads;
  const int kvh = h / P.kv_group;
  const int kind = P.hd[h].kind;
  const int q0 = bq * kBlock;
  const int nrows = min(kBlock, P.s_q - q0);
  const int a0 = q0 + P.s_k - P.s_q;
  const int a1 = a0 + nrows - 1;
  const int last_tile = min(a1 >> 6, P.n_kb - 1);
  const int n_init = P.hd[h].p1;
  const int n_local = P.hd[h].p2;
  TileSeq seq;
  seq.n_kb = P.n_kb;
  seq.list = nullptr;
  seq.any = reinterpret_cast<const int32_t*>(P.q);
  if (kind == KIND_BLOCK) {
    const int64_t base = (int64_t(b) * P.idx_slots + P.hd[h].slot) * P.n_qb + bq;
    const int cnt = max(0, min(load_uniform(P.cnt + base), P.topk_max));
    seq.list = P.idx + base * P.topk_max;
    seq.set({0, 0, 0, 0, 0}, {cnt, 0, 0, 0, 0}, 1);
  } else if (kind == KIND_STREAM) {
    const int lo = min(max(a0 - n_local + 1, 0) >> 6, last_tile + 1);
    const int nsink = min((min(max(n_init, 0), P.s_k) + 63) >> 6, lo);
    seq.set({0, lo, 0, 0, 0}, {nsink, last_tile + 1, 0, 0, 0}, 1);
  } else if (kind == KIND_FULL) {
    seq.set({0, 0, 0, 0, 0}, {P.n_kb, 0, 0, 0, 0}, 1);
  } else {
    seq.set({0, 0, 0, 0, 0}, {last_tile + 1, 0, 0, 0, 0}, 1);
  }
  const int total = seq.total;

  const int64_t bk = int64_t(b) * (P.heads / P.kv_group) + kvh;
  const float vfac = __builtin_amdgcn_ldexpf(1.0f, load_uniform(P.vexp + bk));
  // K is always staged at this head dim (the staging orders each 32-key
  // span's keys for this kernel)
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.kt + bk * P.s_pad * D), short(0), P.s_pad * D * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.vt + bk * P.s_pad * D), short(0), P.s_pad * D * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(reinterpret_cast<const uint16_t*>(P.q) + b * P.q_sb +
                            int64_t(h) * P.q_sh + int64_t(q0) * P.q_ss),
      short(0), int(((nrows - 1) * P.q_ss + D) * 2), 0x00020000);

  // Q rows 16w + lc as the QK B operand (rows past S_q read zeros or rows of
  // the view; their outputs are not stored)
  u32x4 qb[NKS];
  {
    const uint32_t roff = uint32_t((16 * w + lc) * P.q_ss * 2 + 16 * lr);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      qb[ks] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qrs, roff, 64 * ks, 0));
  }
  const float c_log2 = P.hd[h].scale_log2;
  const int ar = a0 + 16 * w + lc;  // absolute position of this lane's row
  const bool is_full = kind == KIND_FULL, is_stream = kind == KIND_STREAM;
  const int key_hi = is_full ? P.s_k - 1 : min(ar, P.s_k - 1);
  const int band_lo = is_stream ? ar - n_local + 1 : 0;
  const int sink_hi = is_stream ? n_init : 0;

  f32x4 o[NDO];
#pragma unroll
  for (int db = 0; db < NDO; ++db) o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m = -1e30f;  // running (biased) max of the row in scaled log2 units
  float l = 0.0f;    // this lane's share of the row sum

  // At D = 256 the workgroup copies each tile's staged K and V into LDS (the
  // four waves read the same operands: each line then leaves L2 once per
  // workgroup instead of once per wave; 64 KB, two workgroups per CU); at
  // D = 512 every wave reads them from L2 itself (a 128 KB tile would leave
  // one workgroup per CU, measured slower).
  constexpr bool SHARED = D == 256;
  constexpr int TILE_BYTES = 64 * D * 2;    // one tile of staged K (or V)
  constexpr int G = TILE_BYTES / 16 / 256;  // 16-byte granules per thread and plane
  __shared__ __align__(16) unsigned char sm[SHARED ? 2 * TILE_BYTES : 16];
  auto lds16 = [&](int off) INLINE -> u32x4 {
    return *reinterpret_cast<const u32x4*>(sm + off);
  };
  // K operand of virtual chunk vc (span vc / 2, half vc % 2) of tile t: the
  // staged chunk 4t + vc, whose row r is key 32 (vc / 2) + 8 (r / 4) +
  // 4 (vc % 2) + r % 4 of the tile; lane (lc, lr) of k-step ks holds
  // elements 32 ks + 8 lr .. +7 of row lc
  auto load_k = [&](int t, int vc, u32x4 (&kr)[NKS]) INLINE {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      if constexpr (SHARED) {
        kr[ks] = lds16((vc * NKS + ks) * 1024 + lane * 16);
      } else {
        const uint32_t vo = uint32_t((4 * t + vc) * NKS * 1024 + lane * 16);
        kr[ks] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, vo, 1024 * ks, 0));
      }
    }
  };
  auto qk = [&](const u32x4 (&kr)[NKS]) INLINE -> f32x4 {
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) acc = mfma_qk<T>(kr[ks], qb[ks], acc);
    return acc;
  };
  // V^T operand (dims 16 db + lc, keys 32 kh + 8 lr .. +7 of tile t) from the
  // staged layout: chunk 4t + 2kh + lr / 2, block db / 2, lane 32 (lr % 2) +
  // 16 (db % 2) + lc
  auto load_v = [&](int t, int kh, u32x4 (&vr)[NDO]) INLINE {
    const int c = 2 * kh + (lr >> 1);  // chunk within the tile
#pragma unroll
    for (int db = 0; db < NDO; ++db) {
      const int go = ((c * NDB + (db >> 1)) * 64 + 32 * (lr & 1) + 16 * (db & 1) + lc) * 16;
      if constexpr (SHARED) {
        vr[db] = lds16(TILE_BYTES + go);
      } else {
        vr[db] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, uint32_t(t * TILE_BYTES + go), 0, 0));
      }
    }
  };

  u32x4 k0[NKS];
  for (int p = 0; p < total; ++p) {
    const int t = seq.template finish<false>(seq.fetch(p));
    if constexpr (SHARED) {
      __syncthreads();  // every wave has read the previous tile
      u32x4 gk[G], gv[G];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const uint32_t go = uint32_t((tid + 256 * u) * 16);
        gk[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, go, t * TILE_BYTES, 0));
        gv[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, go, t * TILE_BYTES, 0));
      }
#pragma unroll
      for (int u = 0; u < G; ++u) {
        *reinterpret_cast<u32x4*>(sm + (tid + 256 * u) * 16) = gk[u];
        *reinterpret_cast<u32x4*>(sm + TILE_BYTES + (tid + 256 * u) * 16) = gv[u];
      }
      __syncthreads();
    }
    // scores of the tile: s[kh][ab] (lane: keys 8 lr + 4 ab + i of span kh)
    f32x4 s[2][2];
    u32x4 vr[NDO];  // V of span 0, requested under the last QK
    load_k(t, 0, k0);
    s[0][0] = qk(k0);
    load_k(t, 1, k0);
    s[0][1] = qk(k0);
    load_k(t, 2, k0);
    s[1][0] = qk(k0);
    load_v(t, 0, vr);
    load_k(t, 3, k0);
    s[1][1] = qk(k0);
    // visibility (every tile: the walk has no separate unmasked part here)
    float mx = -__builtin_inff();
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int ab = 0; ab < 2; ++ab)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 64 * t + 32 * kh + 8 * lr + 4 * ab + i;
          const bool vis = (j <= key_hi) & ((j >= band_lo) | (j < sink_hi));
          const float x = vis ? s[kh][ab][i] : -__builtin_inff();
          s[kh][ab][i] = x;
          mx = fmaxf(mx, x);
        }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx * c_log2 - kPBias);
    if (__ballot(mn != m) != 0) {
      const float al = __builtin_amdgcn_exp2f(m - mn);
      l *= al;
#pragma unroll
      for (int db = 0; db < NDO; ++db) o[db] *= al;
      m = mn;
    }
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      if (kh == 1) load_v(t, 1, vr);  // span 1 into the registers span 0's PV has read
      float pv[2][4];
#pragma unroll
      for (int ab = 0; ab < 2; ++ab)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pv[ab][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kh][ab][i], c_log2, -m));
          l += pv[ab][i];
        }
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      typedef float f2 __attribute__((ext_vector_type(2)));
      const u32x4 pb = u32x4{
          __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{pv[0][0], pv[0][1]}, h2)),
          __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{pv[0][2], pv[0][3]}, h2)),
          __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{pv[1][0], pv[1][1]}, h2)),
          __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{pv[1][2], pv[1][3]}, h2))};
#pragma unroll
      for (int db = 0; db < NDO; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, vr[db]),
                                                       __builtin_bit_cast(f16x8, pb), o[db], 0,
                                                       0, 0);
    }
  }
  // row sum over the row's four lanes; O^T block db: lane l holds dims
  // 16 db + 4 lr .. +3 of row lc
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  const float inv = l > 0.0f ? vfac / l : 0.0f;
  const int row = q0 + 16 * w + lc;
  if (row < P.s_q) {
    const int64_t obase = b * P.o_sb + int64_t(h) * P.o_sh + int64_t(row) * P.o_ss;
#pragma unroll
    for (int db = 0; db < NDO; ++db) {
      const int d = 16 * db + 4 * lr;
      if constexpr (OUT_F32) {
        store_out4<float>(reinterpret_cast<float*>(P.o) + obase + d, o[db][0] * inv,
                          o[db][1] * inv, o[db][2] * inv, o[db][3] * inv);
      } else {
        store_out4_16<T>(reinterpret_cast<uint16_t*>(P.o) + obase + d, o[db][0] * inv,
                         o[db][1] * inv, o[db][2] * inv, o[db][3] * inv);
      }
    }
  }
}

template <typename T, bool OUT_F32, int D>
static hipError_t launch_wide_t(const AttnParams& p, hipStream_t st) {
  int64_t items = int64_t(p.n_qb) * p.batch * p.heads;
  if (p.n_hl) {
    int longest = 0;
    for (int x = 0; x < 8; ++x) longest = p.xcd_count[x] > longest ? p.xcd_count[x] : longest;
    items = 8 * int64_t(longest);
  }
  if (items == 0) return hipSuccess;
  hipLaunchKernelGGL((attn_wide_kernel<T, OUT_F32, D>), dim3(uint32_t(items)), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T, bool OUT_F32, int D, bool VS>
static hipError_t launch_attn_t(const AttnParams& p, hipStream_t st) {
  int64_t items = int64_t(p.n_qb) * p.batch * p.heads;
  if (p.n_hl) {
    int longest = 0;
    for (int x = 0; x < 8; ++x) longest = p.xcd_count[x] > longest ? p.xcd_count[x] : longest;
    items = 8 * int64_t(longest);
  }
  if (VS) {
    // persistent grid: the resident workgroups of every XCD (2 per CU at
    // two waves per SIMD, 1 for D = 128), capped by the work
    const int64_t per_xcd = p.wg_per_xcd * (D > 96 ? 1 : 2);
    items = items < 8 * per_xcd ? items : 8 * per_xcd;
    if (items == 0) return hipSuccess;
    hipLaunchKernelGGL(queue_reset_kernel, dim3(1), dim3(64), 0, st, p.queue);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (items == 0) return hipSuccess;
  hipLaunchKernelGGL((attn_kernel<T, OUT_F32, D, VS>), dim3(uint32_t(items)), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T, bool OUT_F32, bool VS>
static hipError_t launch_attn_d(const AttnParams& p, int D, hipStream_t st) {
  if (D == 256) return VS ? hipErrorInvalidValue : launch_wide_t<T, OUT_F32, 256>(p, st);
  if (D == 512) return VS ? hipErrorInvalidValue : launch_wide_t<T, OUT_F32, 512>(p, st);
  if (D == 64) return launch_attn_t<T, OUT_F32, 64, VS>(p, st);
  if (D == 96) return launch_attn_t<T, OUT_F32, 96, VS>(p, st);
  return launch_attn_t<T, OUT_F32, 128, VS>(p, st);
}

hipError_t launch_attention(const AttnParams& p, int dtype, int out_dtype, int D,
                            hipStream_t st) {
  const bool f32 = out_dtype == 3;
  if (dtype == Bf16::id)
    return f32 ? launch_attn_d<Bf16, true, false>(p, D, st) : launch_attn_d<Bf16, false, false>(p, D, st);
  return f32 ? launch_attn_d<F16, true, false>(p, D, st) : launch_attn_d<F16, false, false>(p, D, st);
}

hipError_t launch_attention_vs(const AttnParams& p, int dtype, int out_dtype, int D,
                               hipStream_t st) {
  const bool f32 = out_dtype == 3;
  if (dtype == Bf16::id)
    return f32 ? launch_attn_d<Bf16, true, true>(p, D, st) : launch_attn_d<Bf16, false, true>(p, D, st);
  return f32 ? launch_attn_d<F16, true, true>(p, D, st) : launch_attn_d<F16, false, true>(p, D, st);
}

}  // namespace msa
