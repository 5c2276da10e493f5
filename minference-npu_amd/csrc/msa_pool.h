// Pooling pass of the block estimator (device code shared by pool_kernel and
// the fused staging launch).
//
// Reference semantics: _select_block_sparse_topk_indices,
// MInference-NPU/minference/ops/block_sparse_kernel_npu.py:240-252: the mean
// of each block of block_size rows (a multiple of 64) in the input dtype (a
// partial last block is zero padded and still divided by block_size), i.e.
// the fp32 sum divided by block_size and rounded to bf16/fp16.  The block
// sums are accumulated in fp64, exact for 16-bit inputs, so the sum does not
// depend on the summation order.
#pragma once

#include "msa_common.h"
#include "msa_kernels.h"

namespace msa {

__host__ __device__ inline int pool_groups(int nb, int per_wg) { return (nb + per_wg - 1) / per_wg; }

// Workgroup g of the pass: the Q groups of every (batch, slot), then the K
// groups of every (batch, distinct kv head).
__host__ __device__ inline int pool_wg_count(const PoolParams& p) {
  return p.batch * (p.n_slots * pool_groups(p.n_qb, p.pool_blocks) +
                    p.n_kvp * pool_groups(p.n_kb, p.pool_blocks));
}

// One workgroup of 256 threads pools blocks blk0 .. blk0 + PB - 1 (those
// below nb) of a [S][D] matrix with row stride ss into dst [nb][D]; thread
// (bg, c) sums 16-byte chunk c of block blk0 + bg over its brows rows (a
// multiple of 8), eight rows' loads in flight, and stores the 8 pooled
// values as one 16-byte chunk.
template <typename T, int D>
__device__ inline void pool_block_group(const uint16_t* base, int64_t ss, int64_t S, int nb,
                                        int blk0, int brows, uint16_t* dst) {
  constexpr int KCH = D / 8;  // 16-byte chunks per row
  constexpr int PB = pool_blocks_for(D);
  static_assert(PB * KCH <= 256, "one thread per (block, chunk)");
  const int t = threadIdx.x;
  const int bg = t / KCH;
  const int c = t - bg * KCH;
  const int blk = blk0 + bg;
  if (bg >= PB || blk >= nb) return;
  double acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0;
  const int64_t row0 = int64_t(blk) * brows;
  const int rows = int(min(int64_t(brows), S - row0));  // rows past S pool as zeros
  const uint16_t* p = base + row0 * ss + c * 8;
  for (int r0 = 0; r0 < rows; r0 += 8) {
    u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = r0 + u < rows ? load16(p + (r0 + u) * ss) : zero_u32x4();
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] += double(T::to_float(uint16_t(v[u][e] & 0xffffu)));
        acc[2 * e + 1] += double(T::to_float(uint16_t(v[u][e] >> 16)));
      }
  }
  // mean: the fp32 sum divided by brows (IEEE division, as torch's mean
  // divides), then rounded to the input dtype
  const float n = float(brows);
  u32x4 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t lo = T::from_float(float(acc[2 * e]) / n);
    const uint32_t hi = T::from_float(float(acc[2 * e + 1]) / n);
    out[e] = lo | (hi << 16);
  }
  store16(dst + int64_t(blk) * D + c * 8, out);
}

// Workgroup g (0 <= g < pool_wg_count(P)) of the pooling pass.
template <typename T, int D>
__device__ inline void pool_workgroup(const PoolParams& P, int g) {
  constexpr int PB = pool_blocks_for(D);
  const int n_qg = pool_groups(P.n_qb, PB);
  const int n_q_wg = P.batch * P.n_slots * n_qg;
  if (g < n_q_wg) {
    const int sb = g / n_qg;  // b * n_slots + slot
    const int grp = g - sb * n_qg;
    const int b = sb / P.n_slots;
    const int head = P.slot_heads[sb - b * P.n_slots];
    const uint16_t* base =
        reinterpret_cast<const uint16_t*>(P.q) + b * P.q_sb + int64_t(head) * P.q_sh;
    pool_block_group<T, D>(base, P.q_ss, P.s_q, P.n_qb, grp * PB, P.pool_rows,
                           P.q_pool + int64_t(sb) * P.n_qb_pad * D);
    return;
  }
  g -= n_q_wg;
  const int n_kg = pool_groups(P.n_kb, PB);
  const int bi = g / n_kg;  // b * n_kvp + i
  const int grp = g - bi * n_kg;
  const int b = bi / P.n_kvp;
  const int i = bi - b * P.n_kvp;
  const uint16_t* base =
      reinterpret_cast<const uint16_t*>(P.k) + b * P.k_sb + int64_t(P.kvp_head[i]) * P.k_sh;
  pool_block_group<T, D>(base, P.k_ss, P.s_k, P.n_kb, grp * PB, P.pool_rows,
                         P.k_pool + (int64_t(b) * P.n_slots + i) * P.n_kb * D);
}

}  // namespace msa
