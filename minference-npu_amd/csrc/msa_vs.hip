// vertical_and_slash: per query block, the key tiles and key masks the
// attention kernel walks.
//
// Reference semantics: _build_vs_mask_direct, MInference-NPU/minference/ops/
// vertical_slash_kernel_npu.py:282-367 (the production path of
// vertical_slash_sparse_attention, :518-599).  Query block bq (rows
// [64 bq, end_m), end_m = 64 (bq + 1)) sees
//   * for every slash s < end_m the 64 keys [hi - 64, hi),
//     hi = clamp(end_m - s, 64, S_k) (lower end clamped to 0),
//   * every vertical column (clamped into [0, S_k)),
// under the causal mask j <= i.
//
// vs_build_kernel turns that into lists per (slot, query block):
//   * key tiles t <= bq that a slash window meets, plus tile bq if a vertical
//     column lies in it; the mask holds the slash keys and the vertical
//     columns of the tile (the kernel adds the causal mask for t == bq);
//   * gathered tiles n_kb + g: vertical columns c in [64 g, 64 g + 64) of
//     the slot's column list that lie before 64 bq in a tile no slash window
//     meets; their K/V rows are staged contiguously (stage_kernel, gather
//     mode) so that scattered columns cost a dense tile, not one tile each.
// The attention kernel's wave w walks the 16-key chunk w of every tile, so
// each wave gets a list of its own: the tiles whose chunk w holds a visible
// key, entry = tile id << 16 | the chunk's 16 key bits.  (A slash window of
// 64 keys meets two tiles but only four or five of their eight chunks.)
// Entries whose 16 keys are all visible to every row (key tiles t < bq and
// gathered tiles, chunk bits all set) come first and run without a mask;
// then the key tiles, then the gathered tiles, that need one.  Every visible
// key appears in exactly one entry of one list.

#include "msa_common.h"
#include "msa_kernels.h"

namespace msa {

constexpr int kVsMaxTiles = kVsMaxSeq / kBlock;

__device__ inline uint64_t bit_range(int a, int b) {  // bits [a, b), 0 <= a < b <= 64
  const uint64_t hi = b >= 64 ? ~0ull : ((1ull << b) - 1ull);
  return hi & ~((1ull << a) - 1ull);
}

__device__ inline void lds_or64(uint32_t* m, int t, uint64_t v) {
  if (uint32_t(v)) atomicOr(&m[2 * t], uint32_t(v));
  if (uint32_t(v >> 32)) atomicOr(&m[2 * t + 1], uint32_t(v >> 32));
}

__device__ inline uint64_t lds_get64(const uint32_t* m, int t) {
  return uint64_t(m[2 * t]) | (uint64_t(m[2 * t + 1]) << 32);
}

// Block-wide exclusive prefixes of N 0/1 flags over 256 threads: pre[i] =
// the flags i of the threads before this one, tot[i] = the block's total.
// scratch: 4 * N ints.
template <int N>
__device__ inline void block_prefix(const bool (&flag)[N], int* scratch, int (&pre)[N],
                                    int (&tot)[N]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint64_t bal = __ballot(flag[i]);
    pre[i] = __popcll(bal & below);
    if (lane == 0) scratch[4 * i + w] = __popcll(bal);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) {
    int before = 0, all = 0;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      before += v < w ? scratch[4 * i + v] : 0;
      all += scratch[4 * i + v];
    }
    pre[i] += before;
    tot[i] = all;
  }
  __syncthreads();
}

// Chunk w of a tile's mask m for wave w's list: 1 = unmasked entry (all 16
// keys visible to every row: a key tile below the block or a gathered
// tile), 2 = masked entry, 0 = no visible key in the chunk.
__device__ inline int chunk_class(uint64_t m, int w, bool below_block) {
  const uint32_t c = uint32_t(m >> (16 * w)) & 0xffffu;
  return c == 0u ? 0 : (c == 0xffffu && below_block ? 1 : 2);
}

__global__ __launch_bounds__(256) void vs_build_kernel(VsBuildParams P) {
  __shared__ uint32_t um[2 * kVsMaxTiles];  // per key tile: slash keys, then vertical keys
  __shared__ uint32_t gm[2 * kVsMaxTiles];  // per gathered tile: gathered columns
  __shared__ int scratch[32];
  const int bq = blockIdx.x;
  const int bs = blockIdx.y;  // b * slots + slot
  const int tid = threadIdx.x;
  const int end_m = kBlock * (bq + 1);
  const int n_t = min(bq + 1, P.n_kb);  // key tiles any row of the block can see
  const int nv = min(max(P.v_cnt[bs], 0), P.v_stride);
  const int ns = min(max(P.s_cnt[bs], 0), P.s_stride);
  const int n_g = (nv + kBlock - 1) / kBlock;
  const int32_t* vrow = P.v_idx + int64_t(bs) * P.v_stride;
  const int32_t* srow = P.s_idx + int64_t(bs) * P.s_stride;

  for (int i = tid; i < 2 * n_t; i += 256) um[i] = 0u;
  for (int i = tid; i < 2 * n_g; i += 256) gm[i] = 0u;
  __syncthreads();

  // slash windows, clipped to the keys the block's rows can reach
  const int kend = min(end_m, P.s_k);
  for (int i = tid; i < ns; i += 256) {
    const int64_t s = srow[i];
    if (s >= end_m) continue;
    const int hi = int(min(max(int64_t(end_m) - s, int64_t(kBlock)), int64_t(P.s_k)));
    const int lo = max(hi - kBlock, 0);
    const int hc = min(hi, kend);
    if (lo >= hc) continue;
    const int t0 = lo / kBlock, t1 = (hc - 1) / kBlock;
    for (int t = t0; t <= t1; ++t)
      lds_or64(um, t, bit_range(max(lo, kBlock * t) - kBlock * t, min(hc, kBlock * t + kBlock) - kBlock * t));
  }
  __syncthreads();

  // vertical columns: into a tile a slash window meets (or the diagonal
  // tile), else into the gathered set.  A tile below bq with no slash key is
  // never written in this phase, so the membership test is stable.
  for (int c = tid; c < nv; c += 256) {
    const int col = min(max(vrow[c], 0), P.s_k - 1);
    if (col >= end_m) continue;
    const int t = col / kBlock;
    if (t == bq || lds_get64(um, t) != 0ull) {
      lds_or64(um, t, 1ull << (col - kBlock * t));
    } else {
      lds_or64(gm, c / kBlock, 1ull << (c % kBlock));
    }
  }
  __syncthreads();

  // pass 1: each wave's count of unmasked entries (key tiles, then gathered)
  const int64_t row = int64_t(bs) * P.n_qb + bq;
  int n_un[4] = {0, 0, 0, 0};
  for (int e0 = 0; e0 < n_t + n_g; e0 += 256) {
    const int e = e0 + tid;
    const bool gat = e >= n_t;
    const uint64_t m = e < n_t ? lds_get64(um, e) : (e < n_t + n_g ? lds_get64(gm, e - n_t) : 0ull);
    const bool below = gat || e < bq;
    bool f[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) f[w] = chunk_class(m, w, below) == 1;
    int pre[4], tot[4];
    block_prefix<4>(f, scratch, pre, tot);
#pragma unroll
    for (int w = 0; w < 4; ++w) n_un[w] += tot[w];
  }
  // pass 2: the entries, unmasked from 0 and masked from n_un[w] in each
  // wave's list
  uint32_t* lists = P.lists + row * 4 * P.cap;
  int off_u[4] = {0, 0, 0, 0}, off_m[4] = {n_un[0], n_un[1], n_un[2], n_un[3]};
  for (int e0 = 0; e0 < n_t + n_g; e0 += 256) {
    const int e = e0 + tid;
    const bool gat = e >= n_t;
    const uint64_t m = e < n_t ? lds_get64(um, e) : (e < n_t + n_g ? lds_get64(gm, e - n_t) : 0ull);
    const bool below = gat || e < bq;
    const uint32_t id = uint32_t(gat ? P.n_kb + (e - n_t) : e) << 16;
    bool f[8];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int c = chunk_class(m, w, below);
      f[w] = c == 1;
      f[4 + w] = c == 2;
    }
    int pre[8], tot[8];
    block_prefix<8>(f, scratch, pre, tot);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t ent = id | (uint32_t(m >> (16 * w)) & 0xffffu);
      if (f[w]) lists[w * P.cap + off_u[w] + pre[w]] = ent;
      if (f[4 + w]) lists[w * P.cap + off_m[w] + pre[4 + w]] = ent;
      off_u[w] += tot[w];
      off_m[w] += tot[4 + w];
    }
  }
  if (tid < 4) {
    P.cnt[2 * (row * 4 + tid)] = n_un[tid];
    P.cnt[2 * (row * 4 + tid) + 1] = off_m[tid];
  }
}

hipError_t launch_vs_build(const VsBuildParams& p, int n_bs, hipStream_t st) {
  hipLaunchKernelGGL(vs_build_kernel, dim3(p.n_qb, n_bs), dim3(256), 0, st, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Estimator: vertical and slash indices of every vertical_and_slash head.
//
// Reference: _vertical_and_slash_kernel, MInference-NPU/minference/modules/
// minference_forward.py:140-165 (LAST_Q = 64, :43; sum_all_diagonal_matrix,
// :124-137).  With n = min(64, S) last query rows:
//   x   = dtype(dtype(q[-n:] . k^T) / sqrt(D))          (bf16/fp16 matmul, then /)
//   x[r][S - n + c] = -inf for c > r                    (:150-151)
//   p   = softmax(x) per row                            (:152)
//   vertical[j] = sum_r p[r][j];     first 30 = +inf    (:154-155)
//   slash[t]    = sum_r p[r][t + 1 - n + r], t < S;   last 100 = +inf (:159-163)
//   v_idx = top-vsize columns, ascending; s_idx = S - 1 - (top-ssize t), descending.
// Arithmetic: the dot products in fp64 (exact for 16-bit operands), rounded
// to fp32 and to the input dtype; the division in fp32 (correctly rounded);
// the softmax and the sums in fp64 (rows added in order r = 0 .. n-1), each
// sum rounded once to fp32; top-k ties go to the lower index.
// ---------------------------------------------------------------------------

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// 16x16x16 MFMA on 16-bit inputs (16 products per output), fp32 accumulation.
// Lane l: A[l % 16][4 (l / 16) + j], B[4 (l / 16) + j][l % 16], C as 16x16x32.
template <typename T>
__device__ inline f32x4 mfma16(u32x2 a, u32x2 b, f32x4 c);
template <>
__device__ inline f32x4 mfma16<Bf16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                   __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}
template <>
__device__ inline f32x4 mfma16<F16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                               __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
}

// Scores of the n last rows against 64 key columns.  Wave w takes rows
// 16w .. 16w+15; per 16-key block, S^T = K . Q^T on the MFMA (lane l: keys
// 4 (l / 16) + i, row l % 16) as 2 D / 32 partial sums of 16 exact products
// each (16x16x16, separate accumulators; a lane's 8 dims of a 32-dim step
// feed two of them), added in fp32, and sum |q_d k_d| on the 16x16x32.
// Whatever order the hardware adds in, a partial is off by at most
// 16 2^-23 times its sum of |products| (fp32 rounding or truncation) and the
// 2 D / 32 - 1 adds by 6 2^-23 sum |q_d k_d| more, so the total is within
// 24 2^-23 sum |q_d k_d| (plus a term for flushed tiny values; the MFMAs keep
// 16-bit denormals, checked on gfx950).  Rounding to the input dtype is
// monotonic: when both ends of that interval round to the same value, it is
// the rounding of the exact dot product (rounded to fp32 first); otherwise
// (about 1 in 40 entries on N(0,1) data) the wave recomputes the dot
// product exactly in fp64, 16 lanes per entry.
template <typename T, int D>
__global__ __launch_bounds__(256) void vs_score_kernel(VsEstParams P) {
  constexpr int NKS = D / 32;
  constexpr int DPL = D / 16;  // dims per lane of an exact dot product
  __shared__ int32_t flist[4][256];  // per wave: flagged (row, key) of a key block
  __shared__ uint16_t fres[4][256];
  const int j0 = blockIdx.x * kBlock;
  const int bs = blockIdx.y;
  const int b = bs / P.n_slots;
  const int h = P.slot_heads[bs - b * P.n_slots];
  const int kvh = h / P.kv_group;
  const int tid = threadIdx.x;
  const int lane = tid & 63, lr = lane >> 4, lc = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = P.n_rows;
  if (16 * w >= n) return;  // no rows for this wave (S < 64)
  const uint16_t* qb = reinterpret_cast<const uint16_t*>(P.q) + b * P.q_sb + int64_t(h) * P.q_sh;
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(P.k) + b * P.k_sb + int64_t(kvh) * P.k_sh;
  const uint32_t kAbs = 0x7fff7fffu;  // clears the sign bit of both 16-bit halves

  const int r = 16 * w + lc;  // this lane's row of the n last rows (B operand)
  const uint16_t* qrow = qb + int64_t(P.s - n + min(r, n - 1)) * P.q_ss;
  u32x4 qa[NKS], qm[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    qa[ks] = r < n ? load16(qrow + 32 * ks + 8 * lr) : zero_u32x4();
#pragma unroll
    for (int e = 0; e < 4; ++e) qm[ks][e] = qa[ks][e] & kAbs;
  }
  const float c1 = 24.0f * 0x1p-23f * 1.01f;
  const float c0 = float(D + 2) * 0x1p-126f;
  uint16_t* xrow = P.x + int64_t(bs) * kBlock * P.s_pad;
#pragma unroll 1
  for (int c = 0; c < 4; ++c) {
    const int key0 = j0 + 16 * c;
    if (key0 >= P.s) break;
    const int ka = min(key0 + lc, P.s - 1);  // A operand: key row of this lane
    const uint16_t* krow = kb + int64_t(ka) * P.k_ss;
    const f32x4 zero = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 part[2 * NKS];
    f32x4 aacc = zero;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const u32x4 kk = load16(krow + 32 * ks + 8 * lr);
      u32x4 km;
#pragma unroll
      for (int e = 0; e < 4; ++e) km[e] = kk[e] & kAbs;
      part[2 * ks] = mfma16<T>(u32x2{kk[0], kk[1]}, u32x2{qa[ks][0], qa[ks][1]}, zero);
      part[2 * ks + 1] = mfma16<T>(u32x2{kk[2], kk[3]}, u32x2{qa[ks][2], qa[ks][3]}, zero);
      aacc = mfma_qk<T>(km, qm[ks], aacc);
    }
    // entries (key0 + 4 lr + i, row r); only existing ones are redone
    uint16_t a16[4];
    uint32_t redo = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = part[0][i];
#pragma unroll
      for (int p = 1; p < 2 * NKS; ++p) v += part[p][i];
      // the +-bnd adds round too: 2 more 2^-23 units of sum |q_d k_d| >= |v|
      const float bnd = __builtin_fmaf(aacc[i], c1 + 2.0f * 0x1p-23f, c0);
      const uint16_t lo = T::from_float(v - bnd), hi = T::from_float(v + bnd);
      a16[i] = T::from_float(v);
      if (lo != hi && r < n && key0 + 4 * lr + i < P.s) redo |= 1u << i;
    }
    // ambiguous entries: a wave-wide list, 16 lanes per exact dot product
    int pos[4], nflag = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool f = (redo >> i) & 1u;
      const uint64_t bal = __ballot(f);
      pos[i] = nflag + __popcll(bal & ((1ull << lane) - 1ull));
      if (f) flist[w][pos[i]] = (r << 17) | (key0 + 4 * lr + i);
      nflag += __popcll(bal);
    }
    if (nflag) {
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      const int grp = lane >> 4, sl = lane & 15;
      for (int e0 = 0; e0 < nflag; e0 += 4) {
        const int e = e0 + grp;
        double dot = 0.0;
        if (e < nflag) {
          const int code = flist[w][e];
          const uint16_t* qe = qb + int64_t(P.s - n + (code >> 17)) * P.q_ss + DPL * sl;
          const uint16_t* ke = kb + int64_t(code & 0x1ffff) * P.k_ss + DPL * sl;
#pragma unroll
          for (int d = 0; d < DPL; d += 2) {
            const uint32_t qw = *reinterpret_cast<const uint32_t*>(qe + d);
            const uint32_t kw = *reinterpret_cast<const uint32_t*>(ke + d);
            dot = __builtin_fma(double(T::to_float(uint16_t(qw & 0xffffu))),
                                double(T::to_float(uint16_t(kw & 0xffffu))), dot);
            dot = __builtin_fma(double(T::to_float(uint16_t(qw >> 16))),
                                double(T::to_float(uint16_t(kw >> 16))), dot);
          }
        }
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
        if (sl == 0 && e < nflag) fres[w][e] = T::from_float(float(dot));
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if ((redo >> i) & 1u) a16[i] = fres[w][pos[i]];
      __builtin_amdgcn_wave_barrier();  // list reused by the next key block
    }
    if (r < n) {
      uint16_t out[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = key0 + 4 * lr + i;
        out[i] = j - (P.s - n) > r ? T::from_float(-__builtin_inff())
                                   : T::from_float(T::to_float(a16[i]) / P.sqrt_d);
      }
      uint16_t* dst = xrow + int64_t(r) * P.s_pad + key0 + 4 * lr;
      if (key0 + 4 * lr + 3 < P.s) {  // 4 keys, 8-byte aligned (s_pad and key0 + 4 lr are)
        *reinterpret_cast<uint2*>(dst) = uint2{uint32_t(out[0]) | (uint32_t(out[1]) << 16),
                                               uint32_t(out[2]) | (uint32_t(out[3]) << 16)};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (key0 + 4 * lr + i < P.s) dst[i] = out[i];
      }
    }
  }
}

__device__ inline double block_reduce(double v, bool is_max, double* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const double o = __shfl_xor(v, off, 64);
    v = is_max ? fmax(v, o) : v + o;
  }
  if (lane == 0) red[w] = v;
  __syncthreads();
  double r = red[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) r = is_max ? fmax(r, red[i]) : r + red[i];
  __syncthreads();
  return r;
}

// Row max and the fp64 sum of exp(x - max) of one estimator row; 16-byte
// loads (8 entries), four in flight per thread; entries past s (the row
// padding) do not count.
template <typename T>
__global__ __launch_bounds__(256) void vs_rowstat_kernel(VsEstParams P) {
  __shared__ double red[4];
  const int r = blockIdx.x;
  const int bs = blockIdx.y;
  const uint16_t* xr = P.x + (int64_t(bs) * kBlock + r) * P.s_pad;
  const int n8 = (P.s + 7) / 8;  // 8-entry groups holding entries < s
  auto entry = [&](const u32x4& v, int g, int e) -> double {
    const uint16_t b = uint16_t(e & 1 ? v[e >> 1] >> 16 : v[e >> 1] & 0xffffu);
    return 8 * g + e < P.s ? double(T::to_float(b)) : -__builtin_inf();
  };
  double m = -__builtin_inf();
  for (int g0 = threadIdx.x; g0 < n8; g0 += 4 * 256) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int g = g0 + 256 * u;
      v[u] = g < n8 ? load16(xr + 8 * g) : zero_u32x4();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int g = g0 + 256 * u;
      if (g < n8)
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmax(m, entry(v[u], g, e));
    }
  }
  m = block_reduce(m, true, red);
  double l = 0.0;
  for (int g0 = threadIdx.x; g0 < n8; g0 += 4 * 256) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int g = g0 + 256 * u;
      v[u] = g < n8 ? load16(xr + 8 * g) : zero_u32x4();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int g = g0 + 256 * u;
      if (g < n8)
#pragma unroll
        for (int e = 0; e < 8; ++e) l += exp(entry(v[u], g, e) - m);
    }
  }
  l = block_reduce(l, false, red);
  if (threadIdx.x == 0) {
    P.rmax[bs * kBlock + r] = float(m);
    P.rsum[bs * kBlock + r] = l;
  }
}

// Column sums and diagonal sums of p, rounded to fp32, with the forced
// entries set to +inf.  Thread t of a block owns column / diagonal
// c0 + t; four rows at a time, the block forms p for columns [c0 - 63,
// c0 + 256) once in LDS, and each thread adds its column's p and its
// diagonal's p (column t + 1 - n + r), rows in order r = 0 .. n-1.
template <typename T>
__global__ __launch_bounds__(256) void vs_sums_kernel(VsEstParams P) {
  constexpr int W = 256 + kBlock - 1;  // columns one block needs per row
  constexpr int RB = 4;                // rows per round
  __shared__ double sm[kBlock], sl[kBlock];  // row max, 1 / row sum
  __shared__ double prow[RB][W];
  const int bs = blockIdx.y;
  const int n = P.n_rows;
  const int tid = threadIdx.x;
  if (tid < n) {
    sm[tid] = double(P.rmax[bs * kBlock + tid]);
    sl[tid] = 1.0 / P.rsum[bs * kBlock + tid];  // p = e * (1 / l): within an ulp of e / l
  }
  const int c0 = blockIdx.x * 256;
  const int t = c0 + tid;
  const uint16_t* x = P.x + int64_t(bs) * kBlock * P.s_pad;
  double cv = 0.0, cs = 0.0;
  for (int r0 = 0; r0 < n; r0 += RB) {
    __syncthreads();  // previous rows consumed (and sm / sl written)
    uint16_t xv[(RB * W + 255) / 256];
#pragma unroll
    for (int u = 0; u < (RB * W + 255) / 256; ++u) {
      const int idx = tid + 256 * u;
      const int rr = idx / W, col = c0 - (kBlock - 1) + (idx - rr * W);
      xv[u] = idx < RB * W && r0 + rr < n && col >= 0 && col < P.s
                  ? x[int64_t(r0 + rr) * P.s_pad + col]
                  : uint16_t(0);
    }
#pragma unroll
    for (int u = 0; u < (RB * W + 255) / 256; ++u) {
      const int idx = tid + 256 * u;
      if (idx >= RB * W) break;
      const int rr = idx / W, col = c0 - (kBlock - 1) + (idx - rr * W);
      const int r = r0 + rr;
      prow[rr][idx - rr * W] = r < n && col >= 0 && col < P.s
                                   ? exp(double(T::to_float(xv[u])) - sm[r]) * sl[r]
                                   : 0.0;
    }
    __syncthreads();
    if (t < P.s) {
#pragma unroll
      for (int rr = 0; rr < RB; ++rr) {
        const int r = r0 + rr;
        if (r < n) {
          cv += prow[rr][tid + kBlock - 1];
          if (r >= n - 1 - t) cs += prow[rr][tid + kBlock - 1 + 1 - n + r];
        }
      }
    }
  }
  if (t >= P.s) return;
  float fv = float(cv), fs = float(cs);
  if (t < 30) fv = __builtin_inff();
  if (t >= P.s - 100) fs = __builtin_inff();
  P.vert[int64_t(bs) * P.s + t] = fv;
  P.slash[int64_t(bs) * P.s + t] = fs;
}

// Block-wide exclusive prefix of a 0/1 flag over NT threads (see
// block_prefix).
template <int NT>
__device__ inline int block_prefix_n(bool flag, int* scratch, int* total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t bal = __ballot(flag);
  const int in_wave = __popcll(bal & ((1ull << lane) - 1ull));
  if (lane == 0) scratch[w] = __popcll(bal);
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    before += v < w ? scratch[v] : 0;
    all += scratch[v];
  }
  __syncthreads();
  *total = all;
  return before + in_wave;
}

// Top-k of one score row (y = 0: vertical, y = 1: slash): the k-th largest
// key T by a 32-step bitwise search (the largest T with at least k keys >= T;
// non-negative floats order like their bits), counting with wave ballots
// (no atomics: the keys share their leading bits), then every key above T and
// the lowest-index keys equal to T, in index order.  The first 64K keys stay
// in registers across the passes.
constexpr int kTopkThreads = 1024;
constexpr int kTopkRegs = 64;  // keys per thread held in registers

__global__ __launch_bounds__(kTopkThreads) void vs_topk_kernel(VsEstParams P) {
  __shared__ int scratch[kTopkThreads / 64];
  const int bs = blockIdx.x;
  const int slot = bs % P.n_slots;
  const bool is_slash = blockIdx.y == 1;
  const uint32_t* keys = reinterpret_cast<const uint32_t*>(is_slash ? P.slash : P.vert) +
                         int64_t(bs) * P.s;
  const int kk0 = is_slash ? P.slot_ssize[slot] : P.slot_vsize[slot];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint32_t kr[kTopkRegs];
#pragma unroll
  for (int m = 0; m < kTopkRegs; ++m) {
    const int i = tid + kTopkThreads * m;
    kr[m] = i < P.s ? keys[i] : 0u;  // 0 never counts: candidates are >= 1
  }
  auto count_ge = [&](uint32_t c) -> int {
    int cnt = 0;
#pragma unroll
    for (int m = 0; m < kTopkRegs; ++m) cnt += int(kr[m] >= c);
    for (int i = tid + kTopkThreads * kTopkRegs; i < P.s; i += kTopkThreads) cnt += int(keys[i] >= c);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) cnt += __shfl_xor(cnt, off, 64);
    if (lane == 0) scratch[w] = cnt;
    __syncthreads();
    int all = 0;
#pragma unroll
    for (int v = 0; v < kTopkThreads / 64; ++v) all += scratch[v];
    __syncthreads();
    return all;
  };
  uint32_t t = 0u;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = t | (1u << bit);
    if (count_ge(cand) >= kk0) t = cand;
  }
  const int need_eq = kk0 - count_ge(t + 1u);  // keys equal to t to take
  int32_t* out = is_slash ? P.s_idx + int64_t(bs) * P.s_stride : P.v_idx + int64_t(bs) * P.v_stride;
  int taken = 0, eq_seen = 0;
  for (int i0 = 0; i0 < P.s; i0 += kTopkThreads) {
    const int i = i0 + tid;
    const uint32_t key = i < P.s ? keys[i] : 0u;
    const bool gt = i < P.s && key > t;
    const bool eq = i < P.s && key == t;
    int n_eq;
    const int eq_rank = eq_seen + block_prefix_n<kTopkThreads>(eq, scratch, &n_eq);
    const bool take = gt || (eq && eq_rank < need_eq);
    int n_take;
    const int pos = taken + block_prefix_n<kTopkThreads>(take, scratch, &n_take);
    if (take) out[pos] = is_slash ? P.s - 1 - i : i;
    taken += n_take;
    eq_seen += n_eq;
  }
  if (tid == 0) (is_slash ? P.s_cnt : P.v_cnt)[bs] = kk0;
}

template <typename T, int D>
static hipError_t launch_vs_est_t(const VsEstParams& p, hipStream_t st) {
  const int n_bs = p.batch * p.n_slots;
  hipLaunchKernelGGL((vs_score_kernel<T, D>), dim3(p.s_pad / kBlock, n_bs), dim3(256), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((vs_rowstat_kernel<T>), dim3(p.n_rows, n_bs), dim3(256), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((vs_sums_kernel<T>), dim3((p.s + 255) / 256, n_bs), dim3(256), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(vs_topk_kernel, dim3(n_bs, 2), dim3(kTopkThreads), 0, st, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_vs_est_d(const VsEstParams& p, int D, hipStream_t st) {
  if (D == 64) return launch_vs_est_t<T, 64>(p, st);
  if (D == 96) return launch_vs_est_t<T, 96>(p, st);
  return launch_vs_est_t<T, 128>(p, st);
}

hipError_t launch_vs_estimate(const VsEstParams& p, int dtype, int D, hipStream_t st) {
  return dtype == Bf16::id ? launch_vs_est_d<Bf16>(p, D, st) : launch_vs_est_d<F16>(p, D, st);
}

}  // namespace msa
