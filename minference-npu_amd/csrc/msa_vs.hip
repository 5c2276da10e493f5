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
//   1. full tiles: key tiles t < bq whose 64 keys are all visible (no mask);
//   2. partial tiles: the other key tiles t <= bq that a slash window meets,
//      plus tile bq if a vertical column lies in it; the mask holds the slash
//      keys and the vertical columns of the tile (the kernel adds the causal
//      mask for t == bq);
//   3. gathered tiles n_kb + g: vertical columns c in [64 g, 64 g + 64) of
//      the slot's column list that lie before 64 bq in a tile no slash window
//      meets; their K/V rows are staged contiguously (stage_kernel, gather
//      mode) so that scattered columns cost a dense tile, not one tile each.
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

  // counts: full and partial key tiles, gathered tiles
  int n_full = 0, n_part = 0, n_gath = 0;
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
    int tot;
    block_prefix(g < n_g && lds_get64(gm, g) != 0ull, scratch, &tot);
    n_gath += tot;
  }

  // write the list
  const int64_t row = int64_t(bs) * P.n_qb + bq;
  int32_t* ids = P.ids + row * P.cap;
  uint64_t* masks = P.masks + row * P.cap;
  int off_full = 0, off_part = n_full;
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
  int off_g = n_full + n_part;
  for (int g0 = 0; g0 < n_g; g0 += 256) {
    const int g = g0 + tid;
    const uint64_t m = g < n_g ? lds_get64(gm, g) : 0ull;
    int tg;
    const int pg = block_prefix(m != 0ull, scratch, &tg);
    if (m != 0ull) {
      ids[off_g + pg] = P.n_kb + g;
      masks[off_g + pg] = m;
    }
    off_g += tg;
  }
  if (tid == 0) {
    P.cnt[2 * row] = n_full;
    P.cnt[2 * row + 1] = n_full + n_part + n_gath;
  }
}

hipError_t launch_vs_build(const VsBuildParams& p, int n_bs, hipStream_t st) {
  hipLaunchKernelGGL(vs_build_kernel, dim3(p.n_qb, n_bs), dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace msa
