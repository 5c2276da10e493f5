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
// Pooling: one workgroup per (block, slot*batch, {q,k}).
// q_pool layout [SB][n_qb][D]  (row major, fp32)
// k_poolT layout [SB][D][n_kb] (transposed so the scorer reads it coalesced)
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void pool_kernel(PoolParams P) {
  constexpr int KCH = D / 8;            // 16-byte chunks per row
  constexpr int ROWS_PER_PASS = 256 / KCH;  // thread rows covered per pass
  __shared__ double part[ROWS_PER_PASS][D];

  const int blk = blockIdx.x;
  const int sb = blockIdx.y;  // slot-major: sb = b * n_slots + s
  const bool is_k = blockIdx.z == 1;
  const int b = sb / P.n_slots;
  const int s = sb - b * P.n_slots;
  const int head = P.slot_heads[s];

  const int64_t S = is_k ? P.s_k : P.s_q;
  const int nb = is_k ? P.n_kb : P.n_qb;
  if (blk >= nb) return;
  const uint16_t* base;
  int64_t ss;
  if (is_k) {
    const int kvh = head / P.kv_group;
    base = reinterpret_cast<const uint16_t*>(P.k) + b * P.k_sb + kvh * P.k_sh;
    ss = P.k_ss;
  } else {
    base = reinterpret_cast<const uint16_t*>(P.q) + b * P.q_sb + head * P.q_sh;
    ss = P.q_ss;
  }

  const int t = threadIdx.x;
  const int c = t % KCH;
  const int r0 = t / KCH;
  double acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0;
  if (r0 < ROWS_PER_PASS) {
    for (int r = r0; r < kBlock; r += ROWS_PER_PASS) {
      const int64_t row = int64_t(blk) * kBlock + r;
      if (row < S) {
        u32x4 v = load16(base + row * ss + c * 8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[2 * e] += double(T::to_float(uint16_t(v[e] & 0xffffu)));
          acc[2 * e + 1] += double(T::to_float(uint16_t(v[e] >> 16)));
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) part[r0][c * 8 + e] = acc[e];
  }
  __syncthreads();
  if (t < D) {
    double sum = 0.0;
    for (int r = 0; r < ROWS_PER_PASS; ++r) sum += part[r][t];
    // mean in fp32 (sum / 64 is exact), then rounded to the input dtype
    const float mean = float(sum) * (1.0f / 64.0f);
    const float pooled = T::to_float(T::from_float(mean));
    if (is_k) {
      P.k_poolT[(int64_t(sb) * D + t) * P.n_kb + blk] = pooled;
    } else {
      P.q_pool[(int64_t(sb) * P.n_qb + blk) * D + t] = pooled;
    }
  }
}

// ---------------------------------------------------------------------------
// Scoring + top-k: one workgroup of 4 waves per (R consecutive q blocks, sb).
// ---------------------------------------------------------------------------
__device__ inline uint32_t order_key(float f) {
  f = f + 0.0f;  // -0 -> +0 so that equal scores compare equal
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ inline int wave_excl_prefix(int v, int lane) {
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  return x - v;
}

// Selects the k largest scores of sc[0..n) (ties -> lower index) and writes
// their indices ascending to out[0..k).  n > k.  hist: 256 ints private to
// the wave.
__device__ void wave_topk(const float* sc, int n, int k, int* hist, int32_t* out, int lane) {
  uint32_t prefix = 0u, pmask = 0u;
  int krem = k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = lane; i < 256; i += 64) hist[i] = 0;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    for (int c = lane; c < n; c += 64) {
      const uint32_t u = order_key(sc[c]);
      if ((u & pmask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // lane l owns the bins 255-4l .. 252-4l (descending)
    int h[4];
    int lsum = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h[e] = hist[255 - 4 * lane - e];
      lsum += h[e];
    }
    const int above = wave_excl_prefix(lsum, lane);
    // the digit lives in the lane where above < krem <= above + lsum
    const bool mine = (above < krem) && (krem <= above + lsum);
    const unsigned long long who = __ballot(mine);
    const int src = who ? __ffsll(who) - 1 : 0;
    int digit = 0, newk = 0;
    if (mine) {
      int acc = above;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (acc + h[e] >= krem) {
          digit = 255 - 4 * lane - e;
          newk = krem - acc;
          break;
        }
        acc += h[e];
      }
    }
    digit = __shfl(digit, src, 64);
    krem = __shfl(newk, src, 64);
    prefix |= uint32_t(digit) << shift;
    pmask |= 255u << shift;
  }
  // prefix is the k-th largest key; krem of its equal keys are taken, lowest ids first
  int written = 0, eq_seen = 0;
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int base = 0; base < n; base += 64) {
    const int c = base + lane;
    const bool valid = c < n;
    const uint32_t u = valid ? order_key(sc[c]) : 0u;
    const bool gt = valid && u > prefix;
    const bool eq = valid && u == prefix;
    const unsigned long long eqm = __ballot(eq);
    const int eq_rank = eq_seen + __popcll(eqm & lt);
    const bool sel = gt || (eq && eq_rank < krem);
    const unsigned long long selm = __ballot(sel);
    const int pos = written + __popcll(selm & lt);
    if (sel && pos < k) out[pos] = c;
    written += __popcll(selm);
    eq_seen += __popcll(eqm);
  }
}

template <int D, int R>
__global__ __launch_bounds__(256) void score_topk_kernel(ScoreParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  double* qp = reinterpret_cast<double*>(smem);                  // [R][D]
  int* hist = reinterpret_cast<int*>(qp + R * D);                // [4][256]
  float* sc = reinterpret_cast<float*>(hist + 4 * 256);          // [R][ncand]

  const int sb = blockIdx.y;
  const int bq0 = blockIdx.x * R;
  const int nrows = min(R, P.n_qb - bq0);
  const int ncand = min(bq0 + nrows, P.n_kb);  // causal candidates of the last row
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int w = t >> 6;

  for (int i = t; i < R * D; i += 256) {
    const int r = i / D, d = i - r * D;
    qp[i] = (r < nrows) ? double(P.q_pool[(int64_t(sb) * P.n_qb + bq0 + r) * D + d]) : 0.0;
  }
  __syncthreads();

  // Each thread scores NC columns (stride 256) at once, NC chosen from the
  // candidate count: the pooled-K loads of a d-chunk are issued together and
  // every pooled-Q value read from LDS serves all NC columns.  Per (row,
  // column) the fp64 FMAs run in d order.
  const float* kT = P.k_poolT + int64_t(sb) * D * P.n_kb;
  auto score = [&](auto nc) {
    constexpr int NC = decltype(nc)::value, DC = 8;
    for (int cb = 0; cb < ncand; cb += 256 * NC) {
      double acc[NC][R];
#pragma unroll
      for (int j = 0; j < NC; ++j)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[j][r] = 0.0;
      for (int d0 = 0; d0 < D; d0 += DC) {
        float kv[NC][DC];
#pragma unroll
        for (int j = 0; j < NC; ++j) {
          const int c = min(cb + t + 256 * j, ncand - 1);
#pragma unroll
          for (int u = 0; u < DC; ++u) kv[j][u] = kT[int64_t(d0 + u) * P.n_kb + c];
        }
#pragma unroll
        for (int u = 0; u < DC; ++u)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const double qv = qp[r * D + d0 + u];
#pragma unroll
            for (int j = 0; j < NC; ++j) acc[j][r] = fma(qv, double(kv[j][u]), acc[j][r]);
          }
      }
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int c = cb + t + 256 * j;
        if (c < ncand)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            // forced ids score +inf: always inside the top-k
            const bool forced = ((P.flags & kSelectForceFirst) && c == 0) ||
                                ((P.flags & kSelectForceDiag) && c == bq0 + r);
            sc[r * ncand + c] = forced ? __builtin_inff() : float(acc[j][r]) * P.scale;
          }
      }
    }
  };
  if (ncand > 512) score(std::integral_constant<int, 4>());
  else if (ncand > 256) score(std::integral_constant<int, 2>());
  else score(std::integral_constant<int, 1>());
  __syncthreads();

  const int topk = P.slot_topk[sb % P.n_slots];
  for (int r = w; r < nrows; r += 4) {
    const int bq = bq0 + r;
    const int n = min(bq + 1, P.n_kb);
    const int cnt = min(topk, n);
    int32_t* out = P.idx + (int64_t(sb) * P.n_qb + bq) * P.topk_max;
    if (n <= topk) {
      for (int c = lane; c < n; c += 64) out[c] = c;
    } else {
      wave_topk(sc + r * ncand, n, topk, hist + w * 256, out, lane);
    }
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
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <typename T, int D>
static hipError_t launch_pool_t(const PoolParams& p, hipStream_t st) {
  dim3 grid(max(p.n_qb, p.n_kb), p.batch * p.n_slots, 2);
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

int score_rows_for(int n_kb) {
  if (n_kb <= 2048) return 8;
  if (n_kb <= 4096) return 4;
  if (n_kb <= 8192) return 2;
  if (n_kb <= 16384) return 1;
  return 0;
}

size_t score_smem_bytes(int R, int D, int n_kb) {
  return size_t(R) * D * sizeof(double) + 4 * 256 * sizeof(int) +
         size_t(R) * size_t(n_kb) * sizeof(float);
}

template <int D, int R>
static hipError_t launch_score_t(const ScoreParams& p, hipStream_t st) {
  const size_t smem = score_smem_bytes(R, D, p.n_kb);
  auto kern = score_topk_kernel<D, R>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, int(smem));
  if (e != hipSuccess) return e;
  dim3 grid((p.n_qb + R - 1) / R, p.batch * p.n_slots);
  hipLaunchKernelGGL(kern, grid, dim3(256), smem, st, p);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_score_d(const ScoreParams& p, int R, hipStream_t st) {
  switch (R) {
    case 8: return launch_score_t<D, 8>(p, st);
    case 4: return launch_score_t<D, 4>(p, st);
    case 2: return launch_score_t<D, 2>(p, st);
    default: return launch_score_t<D, 1>(p, st);
  }
}

hipError_t launch_score(const ScoreParams& p, int D, hipStream_t st) {
  const int R = score_rows_for(p.n_kb);
  if (D == 64) return launch_score_d<64>(p, R, st);
  if (D == 96) return launch_score_d<96>(p, R, st);
  return launch_score_d<128>(p, R, st);
}

}  // namespace msa
