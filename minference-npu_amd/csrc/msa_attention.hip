// Unified tile-list flash attention for one prefill layer (all heads, one grid).
//
// Work item = (head, 64-row query block).  Each item walks a list of 64-key
// tiles whose shape depends on the head kind:
//   dense        : every causal tile 0..diag              (backend_npu/attention.py:192-255)
//   stream_llm   : sink tiles, then the local band tiles  (ops/streaming_kernel_npu.py:94-146)
//   block_sparse : the estimator's block ids              (ops/block_sparse_kernel_npu.py:266-348,
//                                                          ops/tilelang_sparse_attention_h1.py:367-683)
// Token visibility (exact reference masks; row a is the absolute position
// i + S_k - S_q):
//   all kinds : j <= a and j < S_k
//   stream    : and (j > a - n_local or j < n_init)
// Rows with no visible key produce 0 (the reference's nan_to_num).
//
// CDNA4 mapping (one workgroup = 4 wave64 = one 64-row query block):
//   wave w = (row half rh, key half kh) owns query rows [32rh, 32rh+32) and
//   keys [32kh, 32kh+32) of every tile, with a private online-softmax state;
//   the two key halves of a row half merge once at the end.
//   S^T = K.Q^T on v_mfma_f32_32x32x16_{bf16,f16} (A = K tile from LDS,
//   B = Q from registers), so the accumulator layout (one query row per lane)
//   is directly the B operand of O^T = V^T.P^T on v_mfma_f32_32x32x16_f16.
//   P is rounded to fp16 (11-bit mantissa) for the PV product.
//   V is staged once per layer as fp16 V^T with keys permuted inside each
//   16-key group so every PV A operand is one 16-byte LDS read.
//   K and V^T tiles are double-buffered in LDS (XOR-swizzled 16-byte slots,
//   no bank conflicts) and the next tile is prefetched by buffer loads.
//   The running max moves only when a row max grows by more than 2^8, so the
//   O rescale is rare; the row max needs one lane^32 exchange per tile.
//   Tiles that need no mask run first; boundary tiles (diagonal, band start,
//   partial sink, S_k end) run last with the elementwise mask.

#include <type_traits>

#include "msa_common.h"
#include "msa_kernels.h"

namespace msa {

constexpr int KIND_DENSE = 0;
constexpr int KIND_STREAM = 1;
constexpr int KIND_BLOCK = 2;

// Position of key p inside its 16-key group in the staged V^T rows: quads 1
// and 2 are swapped (an involution, so it also maps position -> key).
__device__ inline int vt_perm(int p) {
  const int q = (p >> 2) & 3;
  const int qs = ((q & 1) << 1) | (q >> 1);
  return (p & ~12) | (qs << 2);
}

// ---------------------------------------------------------------------------
// V [B][Hkv][S][D] (bf16/fp16) -> V^T [B*Hkv][D][s_pad] fp16, keys permuted,
// zero padded to s_pad = 64 * n_kb.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void vt_kernel(VtParams P) {
  constexpr int KCH = D / 8;
  constexpr int LP = D + 8;  // padded LDS row (halves)
  __shared__ __align__(16) uint16_t tile[kBlock * LP];
  const int j0 = blockIdx.x * kBlock;
  const int bk = blockIdx.y;  // b * kv_heads + kvh
  const int b = bk / P.kv_heads, kvh = bk - b * P.kv_heads;
  const uint16_t* src = reinterpret_cast<const uint16_t*>(P.v) + b * P.v_sb + kvh * P.v_sh;
  for (int ci = threadIdx.x; ci < kBlock * KCH; ci += 256) {
    const int r = ci / KCH, c = ci - r * KCH;
    const int j = j0 + r;
    u32x4 out = zero_u32x4();
    if (j < P.s_k) {
      const u32x4 in = load16(src + int64_t(j) * P.v_ss + c * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const _Float16 lo = to_f16_sat<T>(uint16_t(in[e] & 0xffffu));
        const _Float16 hi = to_f16_sat<T>(uint16_t(in[e] >> 16));
        out[e] = uint32_t(__builtin_bit_cast(uint16_t, lo)) |
                 (uint32_t(__builtin_bit_cast(uint16_t, hi)) << 16);
      }
    }
    store16(&tile[r * LP + c * 8], out);
  }
  __syncthreads();
  uint16_t* dst = P.vt + int64_t(bk) * D * P.s_pad;
  for (int ci = threadIdx.x; ci < D * 8; ci += 256) {
    const int d = ci >> 3, c = ci & 7;
    u32x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int p0 = c * 8 + 2 * e;
      const uint16_t lo = tile[vt_perm(p0) * LP + d];
      const uint16_t hi = tile[vt_perm(p0 + 1) * LP + d];
      out[e] = uint32_t(lo) | (uint32_t(hi) << 16);
    }
    store16(dst + int64_t(d) * P.s_pad + j0 + c * 8, out);
  }
}

template <typename T, int D>
static hipError_t launch_vt_t(const VtParams& p, hipStream_t st) {
  dim3 grid(p.s_pad / kBlock, p.batch * p.kv_heads);
  hipLaunchKernelGGL((vt_kernel<T, D>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_vt(const VtParams& p, int dtype, int D, hipStream_t st) {
  if (dtype == Bf16::id) {
    if (D == 64) return launch_vt_t<Bf16, 64>(p, st);
    if (D == 96) return launch_vt_t<Bf16, 96>(p, st);
    return launch_vt_t<Bf16, 128>(p, st);
  }
  if (D == 64) return launch_vt_t<F16, 64>(p, st);
  if (D == 96) return launch_vt_t<F16, 96>(p, st);
  return launch_vt_t<F16, 128>(p, st);
}

// ---------------------------------------------------------------------------
// attention
// ---------------------------------------------------------------------------
template <typename T>
__device__ inline f32x16 mfma_qk(u32x4 a, u32x4 b, f32x16 c);

template <>
__device__ inline f32x16 mfma_qk<Bf16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <>
__device__ inline f32x16 mfma_qk<F16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

__device__ inline f32x16 mfma_pv(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// LDS slot swizzles (16-byte granules) that keep the MFMA operand reads free
// of bank conflicts for 8- and 16-lane LDS phases.
__device__ inline int k_swz(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }
__device__ inline int v_swz(int d) { return (d ^ (d >> 3)) & 7; }

// Tile sequence of one work item as up to five segments: the first `nfull`
// segments hold tiles that need no mask, the rest hold the boundary tiles.
// For block_sparse heads the segments index the id list, otherwise they are
// tile numbers.  Segment bounds are wave-uniform (scalar registers).
struct Cursor {
  int lo0, hi0, lo1, hi1, lo2, hi2, lo3, hi3, lo4, hi4;
  int nfull;
  int seg, i, hi;
  int n_kb;
  const int32_t* list;

  __device__ void bounds(int k, int& lo, int& hi_) const {
    lo = k == 0 ? lo0 : k == 1 ? lo1 : k == 2 ? lo2 : k == 3 ? lo3 : lo4;
    hi_ = k == 0 ? hi0 : k == 1 ? hi1 : k == 2 ? hi2 : k == 3 ? hi3 : hi4;
  }
  // next tile (clamped into [0, n_kb) for memory safety) or -1
  __device__ int next(bool& masked) {
    while (i >= hi) {
      if (++seg >= 5) return -1;
      bounds(seg, i, hi);
    }
    masked = seg >= nfull;
    const int t = list ? list[i] : i;
    ++i;
    return min(max(t, 0), n_kb - 1);
  }
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

template <typename T, bool OUT_F32, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void attn_kernel(AttnParams P) {
  constexpr int KCH = D / 8;   // 16-byte chunks per K row
  constexpr int NKS = D / 16;  // QK^T k-steps (16 dims each)
  constexpr int NDB = D / 32;  // PV output blocks of 32 dims
  constexpr int STG = D / 32;  // staged chunks per thread for K and for V^T
  constexpr int K_BYTES = kBlock * D * 2;         // K tile
  constexpr int TILE_BYTES = 2 * K_BYTES;         // K tile + V^T tile
  constexpr int MERGE_BYTES = (2 * NDB * 16 * 64 + 4 * 64) * 4;
  constexpr int LDS_BYTES = 2 * TILE_BYTES > MERGE_BYTES ? 2 * TILE_BYTES : MERGE_BYTES;
  __shared__ __align__(16) unsigned char lds[LDS_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int n = lane & 31;
  const int g = lane >> 5;
  const int w = tid >> 6;
  const int rh = w >> 1;  // query rows 32rh .. 32rh+31
  const int kh = w & 1;   // keys 32kh .. 32kh+31 of every tile

  // ---- work item.  Workgroups are dispatched round-robin over the 8 XCDs;
  // each XCD walks its own heads one at a time (query blocks longest-first),
  // so the K/V of the 8 heads in flight stay resident in L2 / Infinity Cache.
  const int BH = P.batch * P.heads;
  const int item = blockIdx.x;
  int hh, bq;
  if (P.xcd_heads) {
    const int r = item >> 3;
    bq = P.n_qb - 1 - r % P.n_qb;
    hh = P.head_order[(item & 7) * P.xcd_heads + r / P.n_qb];
  } else {
    bq = P.n_qb - 1 - item / BH;
    hh = item % BH;
  }
  const int b = hh / P.heads;
  const int h = hh - b * P.heads;
  const int kvh = h / P.kv_group;
  const HeadArg hd = P.hd[h];
  const int kind = hd.kind;

  const int q0 = bq * kBlock;
  const int nrows = min(kBlock, P.s_q - q0);
  const int off = P.s_k - P.s_q;
  const int a0 = q0 + off;
  const int a1 = q0 + nrows - 1 + off;
  const int last_tile = min(a1 >> 6, P.n_kb - 1);
  const int n_init = hd.p1;
  const int n_local = hd.p2;
  // tile t needs no mask for the causal / S_k bounds iff t < F
  const int Fe = min(min((a0 + 1) >> 6, P.s_k >> 6), last_tile + 1);

  Cursor cur;
  cur.lo0 = cur.hi0 = cur.lo1 = cur.hi1 = cur.lo2 = cur.hi2 = 0;
  cur.lo3 = cur.hi3 = cur.lo4 = cur.hi4 = 0;
  cur.seg = -1;
  cur.i = cur.hi = 0;
  cur.n_kb = P.n_kb;
  cur.list = nullptr;
  if (kind == KIND_BLOCK) {
    // canonical list: ascending causal ids, so the boundary ids come last
    const int64_t base = (int64_t(b) * P.idx_slots + hd.slot) * P.n_qb + bq;
    const int cnt = max(0, min(P.cnt[base], P.topk_max));
    const int32_t* list = P.idx + base * P.topk_max;
    int nf = cnt;
    while (nf > 0 && list[nf - 1] >= Fe) --nf;
    cur.list = list;
    cur.hi0 = nf;
    cur.lo1 = nf;
    cur.hi1 = cnt;
    cur.nfull = 1;
  } else if (kind == KIND_STREAM) {
    const int lo = min(max(a0 - n_local + 1, 0) >> 6, last_tile + 1);
    const int nsink = min((min(max(n_init, 0), P.s_k) + 63) >> 6, lo);
    const int sf = max(0, min(nsink, min(n_init >> 6, Fe)));  // sink tiles below n_init
    int bf0 = a1 - n_local + 1;                                 // band tiles in every row's band
    bf0 = bf0 <= 0 ? 0 : (bf0 + 63) >> 6;
    bf0 = min(max(bf0, lo), last_tile + 1);
    const int fb_hi = max(bf0, Fe);
    cur.hi0 = sf;                       // full sink
    cur.lo1 = bf0; cur.hi1 = fb_hi;     // full band
    cur.lo2 = sf; cur.hi2 = nsink;      // partial sink
    cur.lo3 = lo; cur.hi3 = bf0;        // band tiles cut by the window start
    cur.lo4 = fb_hi; cur.hi4 = last_tile + 1;  // diagonal / S_k boundary
    cur.nfull = 2;
  } else {
    cur.hi0 = Fe;
    cur.lo1 = Fe; cur.hi1 = last_tile + 1;
    cur.nfull = 1;
  }

  const unsigned char* kbytes = reinterpret_cast<const unsigned char*>(P.k) +
                                2 * (b * P.k_sb + int64_t(kvh) * P.k_sh);
  const unsigned char* vtbytes = reinterpret_cast<const unsigned char*>(P.vt) +
                                 2 * ((int64_t(b) * (P.heads / P.kv_group) + kvh) * D * int64_t(P.s_pad));
  const int64_t kss2 = 2 * P.k_ss;

  // ---- Q rows 32rh.. as the B operand: lane (n, g) holds Q[row][16ks + 8g .. +7]
  u32x4 qb[NKS];
  {
    const uint16_t* qbase =
        reinterpret_cast<const uint16_t*>(P.q) + b * P.q_sb + int64_t(h) * P.q_sh;
    const int row = q0 + 32 * rh + n;
#pragma unroll
    for (int kk = 0; kk < NKS; ++kk)
      qb[kk] = row < P.s_q ? load16(qbase + int64_t(row) * P.q_ss + 16 * kk + 8 * g)
                           : zero_u32x4();
  }

  // ---- loop-invariant staging offsets (global bytes within a tile, LDS bytes)
  uint32_t koff[STG], voff[STG], kslot[STG], vslot[STG];
#pragma unroll
  for (int u = 0; u < STG; ++u) {
    const int ci = tid + 256 * u;
    const int r = ci / KCH, c = ci - r * KCH;
    koff[u] = uint32_t(r) * uint32_t(kss2) + 16u * c;
    kslot[u] = 16u * (r * KCH + (c ^ k_swz(r)));
    const int d = ci >> 3, c2 = ci & 7;
    voff[u] = uint32_t(d) * uint32_t(2 * P.s_pad) + 16u * c2;
    vslot[u] = K_BYTES + 16u * (d * 8 + (c2 ^ v_swz(d)));
  }
  // MFMA A-operand LDS offsets: K rows of this lane, V^T rows 32db + n
  const int krow = 32 * kh + n;
  const uint32_t ka0 = 16u * (krow * KCH + (g ^ k_swz(krow)));
  const uint32_t ka1 = 16u * (krow * KCH + ((2 + g) ^ k_swz(krow)));
  uint32_t va[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    const int d = 32 * db + n;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
      va[db][tt] = K_BYTES + 16u * (d * 8 + ((4 * kh + 2 * tt + g) ^ v_swz(d)));
  }

  // Tile staging through buffer loads: the descriptor is rebased on each tile
  // (scalar work) and bounded so that K rows at or past S_k read as zero.
  // Two register sets alternate so each tile is loaded two tiles ahead.
  auto load_tile = [&](int t, u32x4 (&kr)[STG], u32x4 (&vr)[STG]) {
    const int j0 = t * kBlock;
    const int rows = min(kBlock, P.s_k - j0);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(kbytes + int64_t(j0) * kss2), short(0),
        int(rows * kss2), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(vtbytes + 2 * int64_t(j0)), short(0),
        int(D * 2 * P.s_pad - 2 * j0), 0x00020000);
#pragma unroll
    for (int u = 0; u < STG; ++u) {
      kr[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, koff[u], 0, 0));
      vr[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, voff[u], 0, 0));
    }
  };
  auto store_tile = [&](int buf, const u32x4 (&kr)[STG], const u32x4 (&vr)[STG]) {
    unsigned char* base = lds + buf * TILE_BYTES;
#pragma unroll
    for (int u = 0; u < STG; ++u) {
      *reinterpret_cast<u32x4*>(base + kslot[u]) = kr[u];
      *reinterpret_cast<u32x4*>(base + vslot[u]) = vr[u];
    }
  };

  f32x16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
  // m is the running max in scaled log2 units; it only moves when the row
  // max exceeds it by more than 8, so P stays <= 2^8 between rescales.
  float m = -1e30f;
  float l = 0.0f;
  const float c_log2 = hd.scale_log2;
  const int arow = a0 + 32 * rh + n;  // absolute position of this lane's query row
  // per-lane mask bounds: causal and S_k end; the stream band start and sinks
  const int key_hi = min(arow, P.s_k - 1);
  const int band_lo = kind == KIND_STREAM ? arow - n_local + 1 : 0;
  const int sink_hi = kind == KIND_STREAM ? n_init : 0;

  // one tile: QK^T, mask (boundary tiles only), online softmax, PV
  auto step = [&](const unsigned char* tb, int t, bool mt) {

    // S^T[key][row]: 32 keys (this wave's half) x 32 rows
    u32x4 ka[NKS];
#pragma unroll
    for (int kk = 0; kk < NKS; ++kk)
      ka[kk] = *reinterpret_cast<const u32x4*>(tb + ((kk & 1) ? ka1 : ka0) + 64u * (kk >> 1));
    f32x16 s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < NKS; ++kk) s = mfma_qk<T>(ka[kk], qb[kk], s);
    // V^T operands do not depend on P: read them now, under the softmax
    u32x4 vop[NDB][2];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) vop[db][tt] = *reinterpret_cast<const u32x4*>(tb + va[db][tt]);
    __builtin_amdgcn_sched_barrier(0);

    if (mt) {  // visible iff j <= key_hi and (j >= band_lo or j < sink_hi)
      const int jb = t * kBlock + 32 * kh + 4 * g;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int j = jb + 8 * (i >> 2) + (i & 3);
        const bool vis = (j <= key_hi) & ((j >= band_lo) | (j < sink_hi));
        s[i] = vis ? s[i] : -__builtin_inff();
      }
    }
    // row max of the raw scores; lanes n and n+32 hold the two 16-key halves
    // of row n and exchange them with one permlane32 swap
    float mx = fmaxf(fmaxf(s[0], s[1]), s[2]);
#pragma unroll
    for (int i = 3; i < 15; i += 2) mx = fmaxf(fmaxf(mx, s[i]), s[i + 1]);
    mx = fmaxf(mx, s[15]);
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                       false, false);
      mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * c_log2;
    }
    if (__ballot(mx > m + 8.0f)) {  // wave-uniform: some row grew past the slack
      const float mnew = fmaxf(m, mx);
      const float alpha = __builtin_amdgcn_exp2f(m - mnew);
      m = mnew;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
    }
    // P = 2^(s*c - m) rounded to fp16; the row sum uses fp32 P
    u32x4 pb[2];
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], c_log2, -m));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i + 1], c_log2, -m));
      psum += p0 + p1;
      typedef float f2 __attribute__((ext_vector_type(2)));
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      pb[i >> 3][(i & 7) >> 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{p0, p1}, h2));
    }
    l += psum;
    __builtin_amdgcn_sched_barrier(0);
    // O^T[d][row] += V^T[d][key] . P^T[key][row]
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) o[db] = mfma_pv(vop[db][tt], pb[tt], o[db]);

  };

  // Pipeline: tile i is computed from LDS buffer i&1 while tiles i+1 and
  // i+2 are in flight in the two register sets; after the step the set
  // holding tile i+1 is written to the other buffer and reloaded with i+3.
  u32x4 kra[STG], vra[STG], krb[STG], vrb[STG];
  bool mt = false, ma = false, mb = false;
  int t = cur.next(mt);
  if (t >= 0) {
    load_tile(t, kra, vra);
    store_tile(0, kra, vra);
  }
  int ta = cur.next(ma);
  if (ta >= 0) load_tile(ta, kra, vra);
  int tb2 = cur.next(mb);
  if (tb2 >= 0) load_tile(tb2, krb, vrb);
  __syncthreads();
  // Q is complete here; re-define it so no later wait is attributed to its loads.
#pragma unroll
  for (int kk = 0; kk < NKS; ++kk) asm volatile("" : "+v"(qb[kk]));

  while (t >= 0) {
    step(lds, t, mt);
    if (ta < 0) break;
    store_tile(1, kra, vra);
    t = ta;
    mt = ma;
    ta = cur.next(ma);
    if (ta >= 0) load_tile(ta, kra, vra);
    __syncthreads();

    step(lds + TILE_BYTES, t, mt);
    if (tb2 < 0) break;
    store_tile(0, krb, vrb);
    t = tb2;
    mt = mb;
    tb2 = cur.next(mb);
    if (tb2 >= 0) load_tile(tb2, krb, vrb);
    __syncthreads();
  }
  __syncthreads();

  // ---- merge the two key halves of each row half; kh == 0 writes the rows
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  float* mo = reinterpret_cast<float*>(lds);  // [rh][NDB][16][64]
  float* mm = mo + 2 * NDB * 16 * 64;         // [rh][64]
  float* ml = mm + 2 * 64;                    // [rh][64]
  if (kh == 1) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) mo[((rh * NDB + db) * 16 + i) * 64 + lane] = o[db][i];
    mm[rh * 64 + lane] = m;
    ml[rh * 64 + lane] = l;
  }
  __syncthreads();
  if (kh == 1) return;

  const float m_oth = mm[rh * 64 + lane];
  const float l_oth = ml[rh * 64 + lane];
  const float mt2 = fmaxf(m, m_oth);
  const float f0 = __builtin_amdgcn_exp2f(m - mt2);
  const float f1 = __builtin_amdgcn_exp2f(m_oth - mt2);
  const float lt = l * f0 + l_oth * f1;
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  const float s0 = f0 * inv, s1 = f1 * inv;

  const int row = q0 + 32 * rh + n;
  if (row < P.s_q) {
    const int64_t obase = b * P.o_sb + int64_t(h) * P.o_sh + int64_t(row) * P.o_ss;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        float v4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * qd + e;
          v4[e] = o[db][i] * s0 + mo[((rh * NDB + db) * 16 + i) * 64 + lane] * s1;
        }
        const int d = 32 * db + 8 * qd + 4 * g;
        if constexpr (OUT_F32) {
          store_out4<float>(reinterpret_cast<float*>(P.o) + obase + d, v4[0], v4[1], v4[2], v4[3]);
        } else {
          store_out4_16<T>(reinterpret_cast<uint16_t*>(P.o) + obase + d, v4[0], v4[1], v4[2], v4[3]);
        }
      }
    }
  }
}

template <typename T, bool OUT_F32, int D>
static hipError_t launch_attn_t(const AttnParams& p, hipStream_t st) {
  const int64_t items = int64_t(p.n_qb) * p.batch * p.heads;
  hipLaunchKernelGGL((attn_kernel<T, OUT_F32, D>), dim3(uint32_t(items)), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T, bool OUT_F32>
static hipError_t launch_attn_d(const AttnParams& p, int D, hipStream_t st) {
  if (D == 64) return launch_attn_t<T, OUT_F32, 64>(p, st);
  if (D == 96) return launch_attn_t<T, OUT_F32, 96>(p, st);
  return launch_attn_t<T, OUT_F32, 128>(p, st);
}

hipError_t launch_attention(const AttnParams& p, int dtype, int out_dtype, int D,
                            hipStream_t st) {
  const bool f32 = out_dtype == 3;
  if (dtype == Bf16::id)
    return f32 ? launch_attn_d<Bf16, true>(p, D, st) : launch_attn_d<Bf16, false>(p, D, st);
  return f32 ? launch_attn_d<F16, true>(p, D, st) : launch_attn_d<F16, false>(p, D, st);
}

}  // namespace msa
