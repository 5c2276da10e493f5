// Block top-k estimator: 64-token mean pooling of Q/K, pooled scores,
// block-causal mask and per-query-block top-k.
//
// Reference semantics: _select_block_sparse_topk_indices,
// MInference-NPU/minference/ops/block_sparse_kernel_npu.py:230-263.
//   * pooling happens in the input dtype: the fp32 mean of 64 rows (zero rows
//     pad a partial last block, the divisor stays 64) is rounded to bf16/fp16;
//   * scores = q_pool . k_pool * scale in fp32, masked where k_block > q_block;
//   * torch.topk + sort -> the selected causal ids ascending.
// Exactness: the 64-row sums and the 96-term dot products are accumulated in
// fp64.  For 16-bit pooled operands both are exact, so the fp32 score is the
// correctly rounded value whatever the summation order; the CPU oracle uses
// the same rule and the two agree bit for bit.  Ties break to the lower id.

#include <type_traits>

#include "msa_common.h"
#include "msa_kernels.h"

namespace msa {

// ---------------------------------------------------------------------------
// Pooling: one workgroup per (kPoolBlocks consecutive blocks, slot*batch, {q,k}).
// Thread (bg, c) sums 16-byte chunk c of the 64 rows of block blk0 + bg in
// fp64, eight rows' loads in flight.
// q_pool layout [SB][n_qb_pad][D] (row major, fp64: the scorer reads it as
//                                  scalars; rows n_qb .. n_qb_pad-1 unused)
// k_poolT layout [SB][D][n_kb] (transposed so the scorer reads it coalesced;
//                               written through LDS, kPoolBlocks ids per run)
// ---------------------------------------------------------------------------
constexpr int kPoolBlocks = 16;

template <typename T, int D>
__global__ __launch_bounds__(256) void pool_kernel(PoolParams P) {
  constexpr int KCH = D / 8;  // 16-byte chunks per row
  constexpr int G = kPoolBlocks;
  static_assert(G * KCH <= 256, "one thread per (block, chunk)");
  __shared__ float tr[G][D + 1];

  const int sb = blockIdx.y;  // slot-major: sb = b * n_slots + s
  const bool is_k = blockIdx.z == 1;
  const int b = sb / P.n_slots;
  const int s = sb - b * P.n_slots;
  const int head = P.slot_heads[s];
  const int64_t S = is_k ? P.s_k : P.s_q;
  const int nb = is_k ? P.n_kb : P.n_qb;
  const int blk0 = blockIdx.x * G;
  if (blk0 >= nb) return;  // uniform over the workgroup
  const uint16_t* base;
  int64_t ss;
  if (is_k) {
    base = reinterpret_cast<const uint16_t*>(P.k) + b * P.k_sb + (head / P.kv_group) * P.k_sh;
    ss = P.k_ss;
  } else {
    base = reinterpret_cast<const uint16_t*>(P.q) + b * P.q_sb + head * P.q_sh;
    ss = P.q_ss;
  }

  const int t = threadIdx.x;
  const int bg = t / KCH;
  const int c = t - bg * KCH;
  const int blk = blk0 + bg;
  const bool active = bg < G && blk < nb;
  double acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0;
  if (active) {
    const int64_t row0 = int64_t(blk) * kBlock;
    const int rows = int(min(int64_t(kBlock), S - row0));  // rows past S pool as zeros
    const uint16_t* p = base + row0 * ss + c * 8;
    for (int r0 = 0; r0 < kBlock; r0 += 8) {
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
  }
  // mean in fp32 (sum / 64 is exact), then rounded to the input dtype
  float pooled[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) pooled[e] = T::to_float(T::from_float(float(acc[e]) * (1.0f / 64.0f)));
  if (!is_k) {
    if (active) {
      double* dst = P.q_pool + (int64_t(sb) * P.n_qb_pad + blk) * D + c * 8;
#pragma unroll
      for (int e = 0; e < 8; e += 2)
        *reinterpret_cast<double2*>(dst + e) = make_double2(pooled[e], pooled[e + 1]);
    }
    return;
  }
  if (bg < G) {
#pragma unroll
    for (int e = 0; e < 8; ++e) tr[bg][c * 8 + e] = pooled[e];
  }
  __syncthreads();
  const int nvalid = min(G, nb - blk0);
  float* kT = P.k_poolT + int64_t(sb) * D * P.n_kb + blk0;
  for (int i = t; i < D * G; i += 256) {
    const int d = i / G, g = i - d * G;
    if (g < nvalid) kT[int64_t(d) * P.n_kb + g] = tr[g][d];
  }
}

// ---------------------------------------------------------------------------
// Scoring + top-k: one workgroup of 4 waves per (R = 16 consecutive q blocks,
// sb).  Scores: v_mfma_f64_16x16x4f64 tiles of the 16 rows x 16 candidates,
// pooled Q (fp64) as the A operand held in registers, pooled K columns loaded
// coalesced; two independent accumulation chains per wave; every causal
// score goes to the workspace.  Then each wave selects the top-k of its four
// rows: the k-th largest order key by a bitwise search (keys of KPL x 64
// candidates in registers; KPL = 0 reads them from the workspace), stopping
// as soon as a threshold splits off exactly k keys, then an ordered
// compaction, equal keys going to the lower id.
// ---------------------------------------------------------------------------
__device__ inline uint32_t order_key(float f) {
  f = f + 0.0f;  // -0 -> +0 so that equal scores compare equal
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Sum of v over the 64 lanes (every lane active): inclusive scan within the
// 16-lane rows by DPP row shifts, then the row totals by row broadcasts;
// lane 63 holds the total.
__device__ inline int wave_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return __builtin_amdgcn_readlane(v, 63);
}

typedef double f64x4 __attribute__((ext_vector_type(4)));

// Selection of one row: writes the ids of the topk largest keys (equal keys
// to the lower id) ascending to out.  keys(j) = key of candidate 64 j + lane
// (0 past the row), nj key chunks (N > 0: at most N, loop unrolled so that
// register-held keys are indexed statically); T = the k-th largest key or any
// value with exactly topk keys >= T; need_eq = topk - #(keys > T).
template <int N, typename KeyFn>
__device__ inline void emit_topk(KeyFn keys, int nj, uint32_t T, int need_eq, int32_t* out,
                                 int lane) {
  const unsigned long long below = (1ull << lane) - 1ull;
  int written = 0, eq_seen = 0;
  auto one = [&](int j) {
    const uint32_t k = keys(j);
    const bool eq = k == T;
    const unsigned long long eqm = __ballot(eq);
    const bool sel = k > T || (eq && eq_seen + __popcll(eqm & below) < need_eq);
    const unsigned long long selm = __ballot(sel);
    if (sel) out[written + __popcll(selm & below)] = 64 * j + lane;
    written += __popcll(selm);
    eq_seen += __popcll(eqm);
  };
  if constexpr (N > 0) {
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (j < nj) one(j);
  } else {
    for (int j = 0; j < nj; ++j) one(j);
  }
}

// Up to 1024 candidates (KPL <= 16) the kernel fits 128 registers, so four
// workgroups share a CU and a 64K layer's 16 x 64 workgroups are all resident
// at once.
template <int D, int R, int KPL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KPL > 16 ? 1 : 4)))
void score_topk_kernel(ScoreParams P) {
  static_assert(R == 16, "one 16-row fp64 MFMA tile of query blocks, 4 rows per wave");
  constexpr int NK = D / 4;  // k-steps of the 16x16x4 fp64 MFMA

  const int sb = blockIdx.y;
  const int n_groups = (P.n_qb + R - 1) / R;
  // heaviest (last) groups first; every other set of four slots takes the
  // groups in the mirrored order, so that the workgroups dispatched to one CU
  // (ids 256 apart: the same group of four consecutive slots) mix heavy and
  // light groups instead of four copies of one
  const int gx = ((sb >> 2) & 1) ? n_groups - 1 - int(blockIdx.x) : int(blockIdx.x);
  const int bq0 = (n_groups - 1 - gx) * R;
  const int nrows = min(R, P.n_qb - bq0);
  const int ncand = min(bq0 + nrows, P.n_kb);  // causal candidates of the last row
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int w = t >> 6;
  const int l16 = lane & 15;
  const int lq = lane >> 4;
  // row scores of this group: workspace rows [n_qb_pad][n_kb] of the slot
  float* sc = P.scores + (int64_t(sb) * P.n_qb_pad + bq0) * P.n_kb;

  // A operands: pooled Q row bq0 + l16, dims 4s + lq (rows past n_qb are
  // padding, read and never stored)
  double qa[NK];
  {
    const double* qrow = P.q_pool + (int64_t(sb) * P.n_qb_pad + bq0 + l16) * D + lq;
#pragma unroll
    for (int s = 0; s < NK; ++s) qa[s] = qrow[4 * s];
  }
  // candidate tiles of 16 ids, two at a time per wave (independent MFMA
  // chains): wave w takes tiles w + 8 m and w + 8 m + 4.  Output element i
  // of a lane: row lq + 4 i, candidate 16 tile + l16 (the accumulator layout
  // of v_mfma_f64_16x16x4f64, checked on gfx950).
  const float* kT = P.k_poolT + int64_t(sb) * D * P.n_kb + int64_t(lq) * P.n_kb;
  const int n_tiles = (ncand + 15) >> 4;
  auto store = [&](const f64x4& acc, int c) {
    if (c < ncand) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = lq + 4 * i;
        // forced ids score +inf: always inside the top-k
        const bool forced = ((P.flags & kSelectForceFirst) && c == 0) ||
                            ((P.flags & kSelectForceDiag) && c == bq0 + r);
        sc[int64_t(r) * P.n_kb + c] = forced ? __builtin_inff() : float(acc[i]) * P.scale;
      }
    }
  };
  for (int ct = w; ct < n_tiles; ct += 8) {
    const int c0 = ct * 16 + l16;
    const int c1 = c0 + 64;  // tile ct + 4 (may lie past the last tile: clamped, not stored)
    const float* col0 = kT + min(c0, ncand - 1);
    const float* col1 = kT + min(c1, ncand - 1);
    float k0[NK], k1[NK];
#pragma unroll
    for (int s = 0; s < NK; ++s) {
      k0[s] = col0[int64_t(4 * s) * P.n_kb];
      k1[s] = col1[int64_t(4 * s) * P.n_kb];
    }
    f64x4 a0 = {0.0, 0.0, 0.0, 0.0}, a1 = a0;
#pragma unroll
    for (int s = 0; s < NK; ++s) {
      a0 = __builtin_amdgcn_mfma_f64_16x16x4f64(qa[s], double(k0[s]), a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f64_16x16x4f64(qa[s], double(k1[s]), a1, 0, 0, 0);
    }
    store(a0, c0);
    if (ct + 4 < n_tiles) store(a1, c1);
  }
  __syncthreads();

  // ---- top-k, rows 4w .. 4w+3 of the group
  const int topk = P.slot_topk[sb % P.n_slots];
  auto finish_row = [&](int r, bool selected_all) {
    const int bq = bq0 + r;
    const int n = min(bq + 1, P.n_kb);
    const int cnt = min(topk, n);
    int32_t* out = P.idx + (int64_t(sb) * P.n_qb + bq) * P.topk_max;
    if (selected_all)
      for (int c = lane; c < n; c += 64) out[c] = c;
    // Surplus slots (the reference's -inf picks, which torch.topk fills with
    // q-frame future ids): the next ids bq+1, bq+2, ...  The token mask is
    // in the absolute frame (row i at s_k - s_q + i), so with s_q < s_k some
    // of them lie in the past of the block's rows and are attended; the
    // count covers the selected ids plus those surplus ids whose first key
    // is at or before the block's last absolute row.
    for (int p = cnt + lane; p < topk; p += 64) out[p] = bq + 1 + (p - cnt);
    const int a1 = P.s_k - P.s_q + min(64 * bq + 63, P.s_q - 1);
    const int n_sur = max(0, min(topk - cnt, (a1 >> 6) - bq));
    if (lane == 0) P.cnt[int64_t(sb) * P.n_qb + bq] = cnt + n_sur;
  };
  if constexpr (KPL > 0) {
    // the four rows' searches interleaved (independent reduction chains);
    // rows that need no search (n <= topk or past the group) stay done
    uint32_t keys[4][KPL];
    uint32_t T[4];
    bool done[4];
    int nj[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * w + i;
      const int n = r < nrows ? min(bq0 + r + 1, P.n_kb) : 0;
      nj[i] = (n + 63) >> 6;
      done[i] = n <= topk;
      T[i] = 0u;
      const float* row = sc + int64_t(r) * P.n_kb;
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        const int c = 64 * j + lane;
        keys[i][j] = (!done[i] && c < n) ? order_key(row[c]) : 0u;
      }
    }
    for (int bit = 31; bit >= 0; --bit) {
      if (done[0] && done[1] && done[2] && done[3]) break;
      int ge[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t cand = T[i] | (1u << bit);
        int mine = 0;
#pragma unroll
        for (int j = 0; j < KPL; ++j) mine += keys[i][j] >= cand ? 1 : 0;
        ge[i] = wave_sum(mine);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (!done[i]) {
          if (ge[i] >= topk) T[i] = T[i] | (1u << bit);
          if (ge[i] == topk) done[i] = true;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * w + i;
      if (r >= nrows) continue;
      const int n = min(bq0 + r + 1, P.n_kb);
      if (n > topk) {
        int gt = 0;
        if (T[i] != 0xffffffffu) {
#pragma unroll
          for (int j = 0; j < KPL; ++j) gt += keys[i][j] > T[i] ? 1 : 0;
          gt = wave_sum(gt);
        }
        int32_t* out = P.idx + (int64_t(sb) * P.n_qb + bq0 + r) * P.topk_max;
        const uint32_t(&kr)[KPL] = keys[i];
        emit_topk<KPL>([&](int j) { return kr[j]; }, nj[i], T[i], topk - gt, out, lane);
      }
      finish_row(r, n <= topk);
    }
  } else {
    // long key axes: one row at a time, keys read from the workspace
    for (int r = 4 * w; r < min(4 * w + 4, nrows); ++r) {
      const int n = min(bq0 + r + 1, P.n_kb);
      if (n > topk) {
        const float* row = sc + int64_t(r) * P.n_kb;
        auto key_at = [&](int j) -> uint32_t {
          const int c = 64 * j + lane;
          return c < n ? order_key(row[c]) : 0u;
        };
        const int nj = (n + 63) >> 6;
        auto count_ge = [&](uint32_t thr) -> int {
          int mine = 0;
          for (int j = 0; j < nj; ++j) mine += key_at(j) >= thr ? 1 : 0;
          return wave_sum(mine);
        };
        uint32_t T = 0u;
        for (int bit = 31; bit >= 0; --bit) {
          const uint32_t cand = T | (1u << bit);
          const int ge = count_ge(cand);
          if (ge >= topk) T = cand;
          if (ge == topk) break;
        }
        const int need_eq = topk - (T == 0xffffffffu ? 0 : count_ge(T + 1u));
        emit_topk<0>(key_at, nj, T, need_eq,
                  P.idx + (int64_t(sb) * P.n_qb + bq0 + r) * P.topk_max, lane);
      }
      finish_row(r, n <= topk);
    }
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <typename T, int D>
static hipError_t launch_pool_t(const PoolParams& p, hipStream_t st) {
  dim3 grid((max(p.n_qb, p.n_kb) + kPoolBlocks - 1) / kPoolBlocks, p.batch * p.n_slots, 2);
  hipLaunchKernelGGL((pool_kernel<T, D>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_pool(const PoolParams& p, int dtype, int D, hipStream_t st) {
  if (dtype == Bf16::id) {
    if (D == 64) return launch_pool_t<Bf16, 64>(p, st);
    if (D == 96) return launch_pool_t<Bf16, 96>(p, st);
    return launch_pool_t<Bf16, 128>(p, st);
  }
  if (D == 64) return launch_pool_t<F16, 64>(p, st);
  if (D == 96) return launch_pool_t<F16, 96>(p, st);
  return launch_pool_t<F16, 128>(p, st);
}

// Query blocks per scoring workgroup (one 16-row MFMA tile); the row scores
// go to the estimator workspace.
int score_rows_for(int n_kb) { return n_kb <= 16384 ? 16 : 0; }

template <int D, int R, int KPL>
static hipError_t launch_score_t(const ScoreParams& p, hipStream_t st) {
  dim3 grid((p.n_qb + R - 1) / R, p.batch * p.n_slots);
  hipLaunchKernelGGL((score_topk_kernel<D, R, KPL>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

// keys per lane held in registers for the selection: KPL * 64 >= n_kb
template <int D>
static hipError_t launch_score_d(const ScoreParams& p, hipStream_t st) {
  if (p.n_kb <= 256) return launch_score_t<D, 16, 4>(p, st);
  if (p.n_kb <= 512) return launch_score_t<D, 16, 8>(p, st);
  if (p.n_kb <= 1024) return launch_score_t<D, 16, 16>(p, st);
  if (p.n_kb <= 2048) return launch_score_t<D, 16, 32>(p, st);
  return launch_score_t<D, 16, 0>(p, st);
}

hipError_t launch_score(const ScoreParams& p, int D, hipStream_t st) {
  if (D == 64) return launch_score_d<64>(p, st);
  if (D == 96) return launch_score_d<96>(p, st);
  return launch_score_d<128>(p, st);
}

}  // namespace msa
