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
// vs_build_kernel turns that into a list per (slot, query block):
//   * key tiles t <= bq that a slash window meets, plus tile bq if a vertical
//     column lies in it; the mask holds the slash keys and the vertical
//     columns of the tile (the kernel adds the causal mask for t == bq);
//   * gathered tiles n_kb + g: vertical columns c in [64 g, 64 g + 64) of
//     the slot's column list that lie before 64 bq in a tile no slash window
//     meets; their K/V rows are staged contiguously (stage_kernel, gather
//     mode) so that scattered columns cost a dense tile, not one tile each.
// Entries whose 64 keys are all visible to every row (key tiles t < bq with
// a full mask, gathered tiles with a full mask) come first and run without
// a mask; then the key tiles, then the gathered tiles, that need one.
// Every visible key appears in exactly one entry.

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

// Block-wide exclusive prefix of a 0/1 flag over 256 threads; returns the
// prefix and writes the block total to *total.
__device__ inline int block_prefix(bool flag, int* scratch, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t bal = __ballot(flag);
  const int in_wave = __popcll(bal & ((1ull << lane) - 1ull));
  if (lane == 0) scratch[w] = __popcll(bal);
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    before += v < w ? scratch[v] : 0;
    all += scratch[v];
  }
  __syncthreads();
  *total = all;
  return before + in_wave;
}

__global__ __launch_bounds__(256) void vs_build_kernel(VsBuildParams P) {
  __shared__ uint32_t um[2 * kVsMaxTiles];  // per key tile: slash keys, then vertical keys
  __shared__ uint32_t gm[2 * kVsMaxTiles];  // per gathered tile: gathered columns
  __shared__ int scratch[4];
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

  // counts: full and partial key tiles, full and partial gathered tiles
  int n_full = 0, n_part = 0, n_gfull = 0, n_gpart = 0;
  for (int t0 = 0; t0 < n_t; t0 += 256) {
    const int t = t0 + tid;
    const uint64_t m = t < n_t ? lds_get64(um, t) : 0ull;
    const bool full = t < bq && m == ~0ull;
    int tot;
    block_prefix(full, scratch, &tot);
    n_full += tot;
    block_prefix(m != 0ull && !full, scratch, &tot);
    n_part += tot;
  }
  for (int g0 = 0; g0 < n_g; g0 += 256) {
    const int g = g0 + tid;
    const uint64_t m = g < n_g ? lds_get64(gm, g) : 0ull;
    int tot;
    block_prefix(m == ~0ull, scratch, &tot);
    n_gfull += tot;
    block_prefix(m != 0ull && m != ~0ull, scratch, &tot);
    n_gpart += tot;
  }

  // write the list: full key tiles, full gathered tiles | partial key tiles,
  // partial gathered tiles
  const int64_t row = int64_t(bs) * P.n_qb + bq;
  int32_t* ids = P.ids + row * P.cap;
  uint64_t* masks = P.masks + row * P.cap;
  int off_full = 0, off_part = n_full + n_gfull;
  for (int t0 = 0; t0 < n_t; t0 += 256) {
    const int t = t0 + tid;
    const uint64_t m = t < n_t ? lds_get64(um, t) : 0ull;
    const bool full = t < bq && m == ~0ull;
    const bool part = m != 0ull && !full;
    int tf, tp;
    const int pf = block_prefix(full, scratch, &tf);
    const int pp = block_prefix(part, scratch, &tp);
    if (full) {
      ids[off_full + pf] = t;
      masks[off_full + pf] = m;
    } else if (part) {
      ids[off_part + pp] = t;
      masks[off_part + pp] = m;
    }
    off_full += tf;
    off_part += tp;
  }
  int off_gfull = n_full, off_gpart = n_full + n_gfull + n_part;
  for (int g0 = 0; g0 < n_g; g0 += 256) {
    const int g = g0 + tid;
    const uint64_t m = g < n_g ? lds_get64(gm, g) : 0ull;
    const bool full = m == ~0ull;
    const bool part = m != 0ull && !full;
    int tf, tp;
    const int pf = block_prefix(full, scratch, &tf);
    const int pp = block_prefix(part, scratch, &tp);
    if (full) {
      ids[off_gfull + pf] = P.n_kb + g;
      masks[off_gfull + pf] = m;
    } else if (part) {
      ids[off_gpart + pp] = P.n_kb + g;
      masks[off_gpart + pp] = m;
    }
    off_gfull += tf;
    off_gpart += tp;
  }
  if (tid == 0) {
    P.cnt[2 * row] = n_full + n_gfull;
    P.cnt[2 * row + 1] = n_full + n_gfull + n_part + n_gpart;
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

// Scores of the n last rows against 64 key columns: 256 threads, each a 4x4
// block of (row, column) pairs, operands in LDS as fp64.
template <typename T, int D>
__global__ __launch_bounds__(256) void vs_score_kernel(VsEstParams P) {
  constexpr int KP = D + 1;  // padded rows (fp64): the rows a wave reads hit distinct banks
  __shared__ double qs[kBlock * KP];
  __shared__ double ks[kBlock * KP];
  const int j0 = blockIdx.x * kBlock;
  const int bs = blockIdx.y;
  const int b = bs / P.n_slots;
  const int h = P.slot_heads[bs - b * P.n_slots];
  const int kvh = h / P.kv_group;
  const int tid = threadIdx.x;
  const int n = P.n_rows;
  const uint16_t* qb = reinterpret_cast<const uint16_t*>(P.q) + b * P.q_sb + int64_t(h) * P.q_sh;
  const uint16_t* kb = reinterpret_cast<const uint16_t*>(P.k) + b * P.k_sb + int64_t(kvh) * P.k_sh;
  for (int i = tid; i < kBlock * D; i += 256) {
    const int r = i / D, d = i - r * D;
    qs[r * KP + d] = r < n ? double(T::to_float(qb[int64_t(P.s - n + r) * P.q_ss + d])) : 0.0;
    const int j = j0 + r;
    ks[r * KP + d] = j < P.s ? double(T::to_float(kb[int64_t(j) * P.k_ss + d])) : 0.0;
  }
  __syncthreads();
  const int rg = tid >> 4, cg = tid & 15;
  double acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[i][c] = 0.0;
  for (int d = 0; d < D; ++d) {
    double a[4], bb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = qs[(rg + 16 * i) * KP + d];
#pragma unroll
    for (int c = 0; c < 4; ++c) bb[c] = ks[(cg + 16 * c) * KP + d];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[i][c] = __builtin_fma(a[i], bb[c], acc[i][c]);
  }
  uint16_t* xrow = P.x + int64_t(bs) * kBlock * P.s_pad;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = rg + 16 * i;
    if (r >= n) continue;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int j = j0 + cg + 16 * c;
      if (j >= P.s) continue;
      uint16_t out;
      if (j - (P.s - n) > r) {
        out = T::from_float(-__builtin_inff());
      } else {
        const uint16_t a = T::from_float(float(acc[i][c]));
        out = T::from_float(T::to_float(a) / P.sqrt_d);
      }
      xrow[int64_t(r) * P.s_pad + j] = out;
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

// Row max and the fp64 sum of exp(x - max) of one estimator row.
template <typename T>
__global__ __launch_bounds__(256) void vs_rowstat_kernel(VsEstParams P) {
  __shared__ double red[4];
  const int r = blockIdx.x;
  const int bs = blockIdx.y;
  const uint16_t* xr = P.x + (int64_t(bs) * kBlock + r) * P.s_pad;
  double m = -__builtin_inf();
  for (int j = threadIdx.x; j < P.s; j += 256) m = fmax(m, double(T::to_float(xr[j])));
  m = block_reduce(m, true, red);
  double l = 0.0;
  for (int j = threadIdx.x; j < P.s; j += 256) l += exp(double(T::to_float(xr[j])) - m);
  l = block_reduce(l, false, red);
  if (threadIdx.x == 0) {
    P.rmax[bs * kBlock + r] = float(m);
    P.rsum[bs * kBlock + r] = l;
  }
}

// Column sums and diagonal sums of p, rounded to fp32, with the forced
// entries set to +inf.
template <typename T>
__global__ __launch_bounds__(256) void vs_sums_kernel(VsEstParams P) {
  __shared__ double sm[kBlock], sl[kBlock];
  const int bs = blockIdx.y;
  const int n = P.n_rows;
  if (threadIdx.x < n) {
    sm[threadIdx.x] = double(P.rmax[bs * kBlock + threadIdx.x]);
    sl[threadIdx.x] = P.rsum[bs * kBlock + threadIdx.x];
  }
  __syncthreads();
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= P.s) return;
  const uint16_t* x = P.x + int64_t(bs) * kBlock * P.s_pad;
  double cv = 0.0, cs = 0.0;
  for (int r = 0; r < n; ++r) {
    const double p = exp(double(T::to_float(x[int64_t(r) * P.s_pad + t])) - sm[r]) / sl[r];
    cv += p;
  }
  for (int r = max(0, n - 1 - t); r < n; ++r) {
    const int j = t + 1 - n + r;
    cs += exp(double(T::to_float(x[int64_t(r) * P.s_pad + j])) - sm[r]) / sl[r];
  }
  float fv = float(cv), fs = float(cs);
  if (t < 30) fv = __builtin_inff();
  if (t >= P.s - 100) fs = __builtin_inff();
  P.vert[int64_t(bs) * P.s + t] = fv;
  P.slash[int64_t(bs) * P.s + t] = fs;
}

// Top-k of one score row (z = 0: vertical, z = 1: slash): 4-pass MSD radix
// select of the k-th largest key (non-negative floats order like their
// bits), then the keys above it and the lowest-index keys equal to it, in
// index order.
__global__ __launch_bounds__(256) void vs_topk_kernel(VsEstParams P) {
  __shared__ int hist[256];
  __shared__ int sel[2];  // digit, remaining rank
  __shared__ int scratch[4];
  const int bs = blockIdx.x;
  const int slot = bs % P.n_slots;
  const bool is_slash = blockIdx.y == 1;
  const uint32_t* keys = reinterpret_cast<const uint32_t*>(is_slash ? P.slash : P.vert) +
                         int64_t(bs) * P.s;
  const int kk0 = is_slash ? P.slot_ssize[slot] : P.slot_vsize[slot];
  const int tid = threadIdx.x;
  uint32_t prefix = 0u, mask = 0u;
  int kk = kk0;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    hist[tid] = 0;
    __syncthreads();
    for (int i = tid; i < P.s; i += 256) {
      const uint32_t key = keys[i];
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
    }
    __syncthreads();
    if (tid == 0) {
      int cum = 0, digit = 0;
      for (int d = 255; d >= 0; --d) {
        if (cum + hist[d] >= kk) {
          digit = d;
          break;
        }
        cum += hist[d];
      }
      sel[0] = digit;
      sel[1] = kk - cum;
    }
    __syncthreads();
    prefix |= uint32_t(sel[0]) << shift;
    mask |= 255u << shift;
    kk = sel[1];
    __syncthreads();
  }
  // prefix = the k-th largest key; take every key above it and the first kk
  // keys equal to it
  int32_t* out = is_slash ? P.s_idx + int64_t(bs) * P.s_stride : P.v_idx + int64_t(bs) * P.v_stride;
  int taken = 0, eq_seen = 0;
  for (int i0 = 0; i0 < P.s; i0 += 256) {
    const int i = i0 + tid;
    const uint32_t key = i < P.s ? keys[i] : 0u;
    const bool gt = i < P.s && key > prefix;
    const bool eq = i < P.s && key == prefix;
    int n_eq;
    const int eq_rank = eq_seen + block_prefix(eq, scratch, &n_eq);
    const bool take = gt || (eq && eq_rank < kk);
    int n_take;
    const int pos = taken + block_prefix(take, scratch, &n_take);
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
  hipLaunchKernelGGL(vs_topk_kernel, dim3(n_bs, 2), dim3(256), 0, st, p);
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
