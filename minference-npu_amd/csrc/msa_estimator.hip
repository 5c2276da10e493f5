// Block top-k estimator: 64-token mean pooling of Q/K, pooled scores,
// block-causal mask and per-query-block top-k.
//
// Reference semantics: _select_block_sparse_topk_indices,
// MInference-NPU/minference/ops/block_sparse_kernel_npu.py:230-263.
//   * pooling happens in the input dtype: the fp32 mean of 64 rows (zero rows
//     pad a partial last block, the divisor stays 64) is rounded to bf16/fp16
//     (msa_pool.h);
//   * scores = q_pool . k_pool * scale in fp32, masked where k_block > q_block;
//   * torch.topk + sort -> the selected causal ids ascending.
// Exactness: the selection is the top-k of the correctly rounded fp32 scores
// fp32(fp32(q_pool . k_pool) * scale), the exact dot product of the 16-bit
// pooled operands rounded once (the CPU oracle uses the same rule and the two
// agree bit for bit).  Ties break to the lower id; NaN scores rank above
// +inf (torch.topk's order), forced ids above everything.
//
// How the exact selection is reached cheaply: every score is first formed on
// the 16-bit MFMA (fp32 accumulation) together with sum |q_d k_d| on the same
// unit.  The accumulation error of such a product is at most a small multiple
// of 2^-24 * sum |q_d k_d| (plus a term for products below the fp32 normal
// range); e below bounds |exact - approximate| with a 2^11-fold margin over
// the ~100 roundings of a 96-term product.  A bitwise search finds a
// threshold T with exactly k approximate scores >= T.  With s_T its score:
//   approximate > s_T + 2e  -> in the exact top-k (fewer than k candidates
//                              can outrank it: only those counted at T);
//   approximate < s_T - 2e  -> out (all k counted candidates outrank it);
//   otherwise               -> "band": the exact score is recomputed in fp64
//                              and the band's places are filled by exact rank.
// On the benchmark's inputs the band holds one or two candidates per row.
// Rows with a non-finite score or bound take the exact fp64 path for every
// candidate.

#include <type_traits>

#include "msa_common.h"
#include "msa_kernels.h"
#include "msa_pool.h"

namespace msa {

#define INLINE __attribute__((always_inline))

template <typename T, int D>
__global__ __launch_bounds__(256) void pool_kernel(PoolParams P) {
  pool_workgroup<T, D>(P, int(blockIdx.x));
}

int pool_workgroups(const PoolParams& p) { return pool_wg_count(p); }

// ---------------------------------------------------------------------------
// order keys: a uint32 order of the fp32 scores
// ---------------------------------------------------------------------------
constexpr uint32_t kKeyForced = 0xffffffffu;  // forced ids: above everything
constexpr uint32_t kKeyNaN = 0xffc00000u;     // every NaN: above +inf
constexpr uint32_t kKeyInf = 0xff800000u;     // +inf

__device__ inline uint32_t order_key(float f) {
  if (__builtin_isnan(f)) return kKeyNaN;
  f = f + 0.0f;  // -0 -> +0 so that equal scores compare equal
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// inverse of order_key on keys of non-NaN floats
__device__ inline float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ inline int popc_ballot(bool p) { return __popcll(__ballot(p)); }

// f(j) for the key chunks j < nj (nj wave-uniform).  N > 0: register-held
// keys, indexed statically: f runs unconditionally on the first N, N/2 or
// N/4 chunks, the fewest that cover nj (one branch, none per chunk), so f
// must leave chunks past nj as it found them and count nothing there (every
// caller's keys past its row are 0, below every threshold and every
// selection).
template <int N, typename F>
__device__ inline void for_chunks(int nj, F f) {
  if constexpr (N > 0) {
    constexpr int N2 = N / 2 > 0 ? N / 2 : 1;
    constexpr int N4 = N / 4 > 0 ? N / 4 : 1;
    if (nj > N2) {
#pragma unroll
      for (int j = 0; j < N; ++j) f(j);
    } else if (nj > N4) {
#pragma unroll
      for (int j = 0; j < N2; ++j) f(j);
    } else {
#pragma unroll
      for (int j = 0; j < N4; ++j) f(j);
    }
  } else {
    for (int j = 0; j < nj; ++j) f(j);
  }
}

// fp32(fp32(q . k) * scale) with the dot product of the 16-bit rows formed in
// fp64 (exact products; the sum is exact for pooled operands of ordinary
// range).
template <typename T, int D>
__device__ inline float exact_score(const uint16_t* qrow, const uint16_t* krow, float scale) {
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  // two chunks' loads in flight (the callers keep key arrays in registers)
#pragma unroll 2
  for (int c = 0; c < D / 8; ++c) {
    const u32x4 qv = load16(qrow + 8 * c);
    const u32x4 kv = load16(krow + 8 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[e] = __builtin_fma(double(T::to_float(uint16_t(qv[e] & 0xffffu))),
                             double(T::to_float(uint16_t(kv[e] & 0xffffu))), acc[e]);
      acc[e] = __builtin_fma(double(T::to_float(uint16_t(qv[e] >> 16))),
                             double(T::to_float(uint16_t(kv[e] >> 16))), acc[e]);
    }
  }
  return float((acc[0] + acc[1]) + (acc[2] + acc[3])) * scale;
}

// The exact dot product of two 16-bit rows, computed by the 16 lanes of a
// lane row (sl = lane & 15 takes dims D/16 * sl ..) and summed over them; every
// lane of the row returns it.  Products of 16-bit values are exact in fp64 and
// so is the sum for operands of ordinary range, whatever the order: fp32 of it
// is exact_score's dot product.
template <typename T, int D>
__device__ inline double exact_dot16(const uint16_t* qrow, const uint16_t* krow, int sl) {
  constexpr int DPL = D / 16;
  static_assert(DPL % 2 == 0, "whole 32-bit pairs per lane");
  uint32_t qw[DPL / 2], kw[DPL / 2];
#pragma unroll
  for (int i = 0; i < DPL / 2; ++i) {
    qw[i] = *reinterpret_cast<const uint32_t*>(qrow + DPL * sl + 2 * i);
    kw[i] = *reinterpret_cast<const uint32_t*>(krow + DPL * sl + 2 * i);
  }
  double acc = 0.0;
#pragma unroll
  for (int i = 0; i < DPL / 2; ++i) {
    acc = __builtin_fma(double(T::to_float(uint16_t(qw[i] & 0xffffu))),
                        double(T::to_float(uint16_t(kw[i] & 0xffffu))), acc);
    acc = __builtin_fma(double(T::to_float(uint16_t(qw[i] >> 16))),
                        double(T::to_float(uint16_t(kw[i] >> 16))), acc);
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  return acc;
}

// Largest threshold search: starting from T0 (count(keys >= T0) >= topk),
// bits hb .. 0; stops as soon as a threshold counts exactly topk keys.
template <int N, typename Get>
__device__ inline uint32_t search_from(Get get, int nj, int topk, uint32_t T0, int hb) {
  uint32_t T = T0;
  for (int bit = hb; bit >= 0; --bit) {
    const uint32_t cand = T | (1u << bit);
    int ge = 0;
    for_chunks<N>(nj, [&](int j) { ge += popc_ballot(get(j) >= cand); });
    if (ge >= topk) T = cand;
    if (ge == topk) break;
  }
  return T;
}

template <int N, typename Get>
__device__ inline int count_gt(Get get, int nj, uint32_t T) {
  int gt = 0;
  for_chunks<N>(nj, [&](int j) { gt += popc_ballot(get(j) > T); });
  return gt;
}

// Writes the ids of the selection {key > T} + the first need_eq (lowest ids)
// of {key == T} ascending to out.  keys(j) = key of candidate 64 j + lane (0
// past the row; every real key is nonzero and T >= 1).
template <int N, typename Get>
__device__ inline void emit_topk(Get get, int nj, uint32_t T, int need_eq, int32_t* out, int lane) {
  const unsigned long long below = (1ull << lane) - 1ull;
  int written = 0, eq_seen = 0;
  for_chunks<N>(nj, [&](int j) {
    const uint32_t k = get(j);
    const bool eq = k == T;
    const unsigned long long eqm = __ballot(eq);
    const bool sel = k > T || (eq && eq_seen + __popcll(eqm & below) < need_eq);
    const unsigned long long selm = __ballot(sel);
    if (sel) out[written + __popcll(selm & below)] = 64 * j + lane;
    written += __popcll(selm);
    eq_seen += __popcll(eqm);
  });
}

// Writes the ids of the selection {key == kKeyForced} + {chunk j of this
// lane when bit j of selmask is set} ascending to out.
template <int N, typename Get>
__device__ inline void emit_selected(Get get, uint32_t selmask, int nj, int32_t* out, int lane) {
  const unsigned long long below = (1ull << lane) - 1ull;
  int written = 0;
  for_chunks<N>(nj, [&](int j) {
    const bool sel = get(j) == kKeyForced || ((selmask >> (j & 31)) & 1u);
    const unsigned long long selm = __ballot(sel);
    if (sel) out[written + __popcll(selm & below)] = 64 * j + lane;
    written += __popcll(selm);
  });
}

// Band list of a wave: (exact key, candidate id) of the band's members.
constexpr int kBandMax = 64;
struct BandList {
  uint2 m[kBandMax];
  int n;
};

// Fast finish of one row from its approximate keys (forced ids kKeyForced,
// 0 past the row) and a threshold Ta < kKeyForced with count(keys >= Ta)
// >= topk (exactly topk unless the search ran out of bits).  On success the
// keys above the band are kKeyForced, the band's selected members are the
// bits of selmask (N > 0; the keys of those chunks are left as they were) or
// keys set to kKeyForced (N = 0), and every other key is 0: the selection is
// emit_selected's.  Returns false when the row needs the exact path (a
// non-finite score or bound, or more than kBandMax band members); the keys
// may then already be partly rewritten (above the band: kKeyForced, which
// the exact path keeps as selected; below: 0, rescored there).
template <typename T, int D, int N, typename Get, typename Set>
__device__ inline bool finish_fast(Get get, Set set, int n, int nj, int topk, uint32_t Ta, bool fin,
                                   float amax, float scale, const uint16_t* qrow,
                                   const uint16_t* kbase, int lane, BandList& bl,
                                   uint32_t& selmask) {
  const float cm = scale * amax;
  if (!(fin && Ta < kKeyInf && __builtin_isfinite(4.0f * amax) && __builtin_isfinite(4.0f * cm)))
    return false;
  // |exact - approximate| <= e (see the file comment); band half-width 2e
  const float e = (cm * 0x1p-13f + scale * 0x1p-119f) + 0x1p-148f;
  const float e2 = 2.0f * e;
  const float sT = key_float(Ta);
  int nU = 0, nB = 0;
  uint32_t bandmask = 0u;  // N > 0: chunks where this lane's candidate is in the band
  if (lane == 0) bl.n = 0;
  __builtin_amdgcn_wave_barrier();
  for_chunks<N>(nj, [&](int j) {
    const int c = 64 * j + lane;
    const uint32_t k = get(j);
    const bool valid = c < n;
    const bool forced = k == kKeyForced;
    const float d = key_float(k) - sT;
    const bool up = valid && (forced || d > e2);
    const bool band = valid && !forced && !(d > e2) && !(d < -e2);
    set(j, up ? kKeyForced : (band ? k : 0u));
    if constexpr (N > 0) {
      bandmask |= band ? (1u << j) : 0u;
    } else if (band) {
      const int slot = atomicAdd(&bl.n, 1);
      if (slot < kBandMax)
        bl.m[slot] = make_uint2(order_key(exact_score<T, D>(qrow, kbase + int64_t(c) * D, scale)),
                                uint32_t(c));
    }
    nU += popc_ballot(up);
    nB += popc_ballot(band);
  });
  const int need = topk - nU;
  selmask = 0u;
  if (need <= 0) return true;  // exactly topk above the band
  if (need == nB) {            // the whole band
    if constexpr (N > 0) {
      selmask = bandmask;
    } else {
      for_chunks<N>(nj, [&](int j) {
        const uint32_t k = get(j);
        if (k != 0u && k != kKeyForced) set(j, kKeyForced);
      });
    }
    return true;
  }
  if (nB > kBandMax) return false;
  if constexpr (N > 0) {
    // the band's candidates (one or two per row in practice) into the list,
    // then their exact keys, 16 lanes per candidate
    uint32_t bm = bandmask;
    while (bm) {
      const int j = __builtin_ctz(bm);
      bm &= bm - 1u;
      const int slot = atomicAdd(&bl.n, 1);
      bl.m[slot] = make_uint2(0u, uint32_t(64 * j + lane));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int m0 = 0; m0 < nB; m0 += 4) {
      const int m = m0 + (lane >> 4);
      const double dot = exact_dot16<T, D>(qrow, kbase + int64_t(bl.m[min(m, nB - 1)].y) * D,
                                           lane & 15);
      if ((lane & 15) == 0 && m < nB) bl.m[m].x = order_key(float(dot) * scale);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // exact rank among the band (ties: lower id first); the best `need` win
  bool win = false;
  uint32_t my_id = 0xffffffffu;
  if (lane < nB) {
    const uint2 me = bl.m[lane];
    int rank = 0;
    for (int t = 0; t < nB; ++t) {
      const uint2 o = bl.m[t];
      rank += (o.x > me.x || (o.x == me.x && o.y < me.y)) ? 1 : 0;
    }
    win = rank < need;
    my_id = me.y;
  }
  // the band's members mark their candidates: lane (id & 63), chunk (id >> 6)
  for (int t = 0; t < nB; ++t) {
    const int id = __shfl(int(my_id), t, 64);
    const bool w_t = __shfl(int(win), t, 64) != 0;
    if ((id & 63) == lane) {
      if constexpr (N > 0) {
        selmask |= w_t ? 1u << (id >> 6) : 0u;
      } else {
        set(id >> 6, w_t ? kKeyForced : 0u);
      }
    }
  }
  return true;
}

// Exact finish of one row whose keys are in memory (rk[c], c < n; forced ids
// kKeyForced): every other candidate rescored in fp64, then the search.
template <typename T, int D>
__device__ inline void finish_exact(uint32_t* rk, int n, int topk, float scale,
                                    const uint16_t* qrow, const uint16_t* kbase, int lane,
                                    uint32_t& Tf, int& need_eq) {
  const int nj = (n + 63) >> 6;
  auto get = [&](int j) -> uint32_t {
    const int c = 64 * j + lane;
    return c < n ? rk[c] : 0u;
  };
  for (int c = lane; c < n; c += 64)
    if (rk[c] != kKeyForced) rk[c] = order_key(exact_score<T, D>(qrow, kbase + int64_t(c) * D, scale));
  Tf = search_from<0>(get, nj, topk, 0u, 31);
  need_eq = topk - count_gt<0>(get, nj, Tf);
}

// ---------------------------------------------------------------------------
// Scoring + top-k: one workgroup of 4 waves per (16 q blocks, slot): eight
// from each end of the block range, so that workgroups carry equal work.
// Scores: v_mfma_f32_16x16x32 tiles of 16 candidates x 16 rows, the
// pooled K chunk as the A operand, pooled Q (held in registers) as B, plus
// the same product of the magnitudes; wave w takes candidate tiles w, w + 4,
// ...; the fp32 scores (times the scale) go to the workspace, the per-row
// maximum of sum |q_d k_d| to LDS.  Then each wave selects the top-k of its
// four rows: keys of KPL x 64 candidates in registers (KPL = 0: in the
// workspace row, for long key axes), the bitwise searches of two or four
// rows interleaved and bounded by the rows' candidate chunks, then
// finish_fast (or finish_exact) and an ordered compaction.
// ---------------------------------------------------------------------------
template <typename T, int D, int KPL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KPL > 16 || D > 128 ? 1 : 4)))
void score_topk_kernel(ScoreParams P) {
  constexpr int NKS = D / 32;  // k-steps of the 16x16x32 MFMA
  constexpr uint32_t kAbs = 0x7fff7fffu;
  __shared__ uint32_t s_amax[16];
  __shared__ BandList s_band[4];

  const int sb = blockIdx.y;
  // Row slots: 16 query blocks per workgroup, the first halves of groups x
  // and G-1-x (16-block groups) or their second halves, so that every
  // workgroup (and every wave: two rows of each group) holds about the same
  // number of causal candidates.
  const int G = (P.n_qb + 15) / 16;
  const int x = int(blockIdx.x);
  int gA = x, hA = 0, gB = G - 1 - x, hB = 0;
  if (2 * x > G - 1) {
    gA = G - 1 - x;
    hA = 1;
    gB = x;
    hB = 1;
  } else if (2 * x == G - 1) {  // middle group of an odd count: both its halves
    gB = x;
    hB = 1;
  }
  auto row_of = [&](int j) { return j < 8 ? 16 * gA + 8 * hA + j : 16 * gB + 8 * hB + (j - 8); };
  const int rmax = min(row_of(15), P.n_qb - 1);
  const int ncand = min(rmax + 1, P.n_kb);  // causal candidates of the heaviest row
  const int t = threadIdx.x;
  const int lane = t & 63;
  // wave-uniform, so that the rows and their chunk counts are scalar values
  // and the chunk loops branch once, not per lane
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  const int l16 = lane & 15;
  const int lq = lane >> 4;
  const int b = sb / P.n_slots;
  const int slot = sb - b * P.n_slots;
  const uint16_t* qp = P.q_pool + int64_t(sb) * P.n_qb_pad * D;
  const uint16_t* kp = P.k_pool + (int64_t(b) * P.n_slots + P.slot_kvp[slot]) * P.n_kb * D;
  float* sc = P.scores + int64_t(sb) * P.n_qb_pad * P.n_kb_pad;

  if (t < 16) s_amax[t] = 0u;
  // B operands: pooled Q of slot l16's row, dims 32 ks + 8 lq .. +7 (rows
  // past n_qb are padding: read, never used), and their magnitudes
  u32x4 qb[NKS], qa[NKS];
  const int qrow_l = row_of(l16);
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    qb[ks] = load16(qp + int64_t(qrow_l) * D + 32 * ks + 8 * lq);
#pragma unroll
    for (int e = 0; e < 4; ++e) qa[ks][e] = qb[ks][e] & kAbs;
  }
  __syncthreads();

  const int n_tiles = (ncand + 15) >> 4;
  auto load_tile = [&](int ct, u32x4 (&ka)[NKS]) {
    const int cl = min(ct * 16 + l16, ncand - 1);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) ka[ks] = load16(kp + int64_t(cl) * D + 32 * ks + 8 * lq);
  };
  // a lane holds row l16 and candidates 16 ct + 4 lq .. +3 of each tile;
  // wave w scores tiles w, w + 4, ..., two per step, the next two's K
  // operands in flight (clamped tiles past the end are loaded, not stored)
  uint32_t amax_bits = 0u;
  auto score_tile = [&](int ct, const u32x4 (&ka)[NKS]) {
    f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f}, a = s;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) s = mfma_qk<T>(ka[ks], qb[ks], s);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      u32x4 kabs;
#pragma unroll
      for (int e = 0; e < 4; ++e) kabs[e] = ka[ks][e] & kAbs;
      a = mfma_qk<T>(kabs, qa[ks], a);
    }
    const int c = ct * 16 + 4 * lq;
    if (ct < n_tiles && c <= qrow_l && c < ncand)
      *reinterpret_cast<float4*>(sc + int64_t(qrow_l) * P.n_kb_pad + c) =
          make_float4(s[0] * P.scale, s[1] * P.scale, s[2] * P.scale, s[3] * P.scale);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // magnitudes are >= 0: their bits order as integers; a non-finite
      // sum makes the row's bound infinite
      const uint32_t ab = __builtin_isfinite(a[i]) ? __float_as_uint(a[i]) : 0x7f800000u;
      amax_bits = max(amax_bits, ab);
    }
  };
  {
    u32x4 k0[NKS], k1[NKS], n0[NKS], n1[NKS];
    int ct = w;
    if (ct < n_tiles) {
      load_tile(ct, k0);
      load_tile(ct + 4, k1);
    }
    for (; ct < n_tiles; ct += 8) {
      if (ct + 8 < n_tiles) {
        load_tile(ct + 8, n0);
        load_tile(ct + 12, n1);
      }
      score_tile(ct, k0);
      score_tile(ct + 4, k1);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        k0[ks] = n0[ks];
        k1[ks] = n1[ks];
      }
    }
  }
  atomicMax(&s_amax[l16], amax_bits);
  __syncthreads();

  // ---- top-k: wave w takes the rows of slots 2w, 2w+1 (lighter half) and
  // 2w+8, 2w+9 (heavier half); rows are absolute query-block indices
  const int topk = P.slot_topk[slot];
  auto wave_slot = [&](int ii) { return ii < 2 ? 2 * w + ii : 6 + 2 * w + ii; };
  const bool force_first = (P.flags & kSelectForceFirst) != 0;
  const bool force_diag = (P.flags & kSelectForceDiag) != 0;
  auto finish_row = [&](int bq, bool selected_all) {
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
    const int a1 = P.s_k - P.s_q + min(P.block * bq + P.block - 1, P.s_q - 1);
    const int n_sur = max(0, min(topk - cnt, a1 / P.block - bq));
    if (lane == 0) P.cnt[int64_t(sb) * P.n_qb + bq] = cnt + n_sur;
  };
  // approximate key of candidate c of row r (forced ids above everything)
  auto approx_key = [&](int r, int c, bool& nonfinite) -> uint32_t {
    const float a = sc[int64_t(r) * P.n_kb_pad + c];
    const bool forced = (force_first && c == 0) || (force_diag && c == r);
    nonfinite = !forced && !__builtin_isfinite(a);
    return forced ? kKeyForced : order_key(a);
  };
  auto row_out = [&](int r) { return P.idx + (int64_t(sb) * P.n_qb + r) * P.topk_max; };
  auto qrow_of = [&](int r) { return qp + int64_t(r) * D; };

  // row r's keys in the workspace (over its scores), for the exact path
  auto row_keys = [&](int r) { return reinterpret_cast<uint32_t*>(sc + int64_t(r) * P.n_kb_pad); };

  if constexpr (KPL > 0) {
    // rows per pass: the wave's four rows interleaved, or from 1024
    // candidates on two at a time, the lighter pair first (the keys of four
    // rows would not fit the registers)
    constexpr int RP = KPL >= 16 ? 2 : 4;
    for (int p0 = 0; p0 < 4; p0 += RP) {
      uint32_t keys[RP][KPL];
      uint32_t Ta[RP];
      bool done[RP], fin[RP], slow[RP];
      int n[RP], nj[RP];
      int njmax = 0;
      // per row i a compile-time index, so that keys[i][j] stays in registers
      auto each_row = [&](auto f) {
        f(std::integral_constant<int, 0>());
        f(std::integral_constant<int, 1>());
        if constexpr (RP > 2) {
          f(std::integral_constant<int, 2>());
          f(std::integral_constant<int, 3>());
        }
      };
      each_row([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        const int r = row_of(wave_slot(p0 + i));
        n[i] = r < P.n_qb ? min(r + 1, P.n_kb) : 0;
        nj[i] = (n[i] + 63) >> 6;
        done[i] = n[i] <= topk;
        slow[i] = false;
        njmax = done[i] ? njmax : max(njmax, nj[i]);
        Ta[i] = 0u;
        bool nonfin = false;
#pragma unroll
        for (int j = 0; j < KPL; ++j) keys[i][j] = 0u;
        if (!done[i]) {
          // every chunk's load first (clamped into the row), then the keys
          const float* row = sc + int64_t(r) * P.n_kb_pad;
          float a[KPL];
#pragma unroll
          for (int j = 0; j < KPL; ++j) a[j] = row[min(64 * j + lane, n[i] - 1)];
#pragma unroll
          for (int j = 0; j < KPL; ++j) {
            const int c = 64 * j + lane;
            const bool forced = (force_first && c == 0) || (force_diag && c == r);
            nonfin |= c < n[i] && !forced && !__builtin_isfinite(a[j]);
            keys[i][j] = c < n[i] ? (forced ? kKeyForced : order_key(a[j])) : 0u;
          }
        }
        fin[i] = __ballot(nonfin) == 0ull;
      });
      // the pass's searches interleaved (independent reduction chains);
      // rows that need no search (n <= topk or past the group) stay done.
      // Each round counts a fixed number of chunks, NB (KPL, KPL/2 or KPL/4,
      // the smallest that covers the pass's rows), without a branch per
      // chunk: keys past a row are 0 and every candidate is at least 1.
      auto search = [&](auto nbc) INLINE {
        constexpr int NB = decltype(nbc)::value;
        for (int bit = 31; bit >= 0; --bit) {
          bool all_done = true;
#pragma unroll
          for (int i = 0; i < RP; ++i) all_done = all_done && done[i];
          if (all_done) break;
          int ge[RP];
          each_row([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            const uint32_t cand = Ta[i] | (1u << bit);
            int c = 0;
#pragma unroll
            for (int j = 0; j < NB; ++j) c += popc_ballot(keys[i][j] >= cand);
            ge[i] = c;
          });
#pragma unroll
          for (int i = 0; i < RP; ++i) {
            if (!done[i]) {
              if (ge[i] >= topk) Ta[i] = Ta[i] | (1u << bit);
              if (ge[i] == topk) done[i] = true;
            }
          }
        }
      };
      constexpr int NB4 = KPL / 4 > 0 ? KPL / 4 : 1;
      if (njmax > KPL / 2) search(std::integral_constant<int, KPL>());
      else if (njmax > NB4) search(std::integral_constant<int, (KPL / 2 > 0 ? KPL / 2 : 1)>());
      else search(std::integral_constant<int, NB4>());
      each_row([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        const int r = row_of(wave_slot(p0 + i));
        if (r >= P.n_qb || n[i] <= topk) return;
        auto get = [&](int j) -> uint32_t { return keys[i][j]; };
        auto set = [&](int j, uint32_t v) { keys[i][j] = v; };
        uint32_t selmask = 0u;
        if (Ta[i] != kKeyForced &&
            finish_fast<T, D, KPL>(get, set, n[i], nj[i], topk, Ta[i], fin[i],
                                   __uint_as_float(s_amax[wave_slot(p0 + i)]), P.scale, qrow_of(r),
                                   kp, lane,
                                   s_band[w], selmask)) {
          emit_selected<KPL>(get, selmask, nj[i], row_out(r), lane);
        } else if (Ta[i] == kKeyForced) {  // at least topk forced ids: the lowest of them
          emit_topk<KPL>(get, nj[i], kKeyForced, topk, row_out(r), lane);
        } else {
          // exact path, below: the row's approximate keys go to the workspace
          uint32_t* rk = row_keys(r);
          for_chunks<KPL>(nj[i], [&](int j) {
            const int c = 64 * j + lane;
            if (c < n[i]) rk[c] = keys[i][j];
          });
          slow[i] = true;
        }
      });
      for (int i = 0; i < RP; ++i) {
        const int r = row_of(wave_slot(p0 + i));
        if (r >= P.n_qb) continue;
        if (slow[i]) {
          uint32_t Tf;
          int need_eq;
          finish_exact<T, D>(row_keys(r), n[i], topk, P.scale, qrow_of(r), kp, lane, Tf, need_eq);
          uint32_t* rk = row_keys(r);
          const int nn = n[i];
          emit_topk<0>([&](int j) -> uint32_t {
            const int c = 64 * j + lane;
            return c < nn ? rk[c] : 0u;
          }, nj[i], Tf, need_eq, row_out(r), lane);
        }
        finish_row(r, n[i] <= topk);
      }
    }
  } else {
    // long key axes: one row at a time; the row's keys replace its scores in
    // the workspace (the row belongs to this wave)
    for (int ii = 0; ii < 4; ++ii) {
      const int r = row_of(wave_slot(ii));
      if (r >= P.n_qb) continue;
      const int n = min(r + 1, P.n_kb);
      if (n > topk) {
        uint32_t* rk = row_keys(r);
        const int nj = (n + 63) >> 6;
        bool nonfin = false;
        for (int c = lane; c < n; c += 64) {
          bool nf = false;
          rk[c] = approx_key(r, c, nf);
          nonfin |= nf;
        }
        const bool fin = __ballot(nonfin) == 0ull;
        auto get = [&](int j) -> uint32_t {
          const int c = 64 * j + lane;
          return c < n ? rk[c] : 0u;
        };
        auto set = [&](int j, uint32_t v) {
          const int c = 64 * j + lane;
          if (c < n) rk[c] = v;
        };
        const uint32_t Ta = search_from<0>(get, nj, topk, 0u, 31);
        uint32_t selmask = 0u;
        if (Ta == kKeyForced) {  // at least topk forced ids: the lowest of them
          emit_topk<0>(get, nj, kKeyForced, topk, row_out(r), lane);
        } else if (finish_fast<T, D, 0>(get, set, n, nj, topk, Ta, fin,
                                        __uint_as_float(s_amax[wave_slot(ii)]), P.scale,
                                        qrow_of(r), kp, lane, s_band[w], selmask)) {
          emit_selected<0>(get, 0u, nj, row_out(r), lane);
        } else {
          uint32_t Tf;
          int need_eq;
          finish_exact<T, D>(rk, n, topk, P.scale, qrow_of(r), kp, lane, Tf, need_eq);
          emit_topk<0>(get, nj, Tf, need_eq, row_out(r), lane);
        }
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
  const int n = pool_wg_count(p);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL((pool_kernel<T, D>), dim3(n), dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_pool(const PoolParams& p, int dtype, int D, hipStream_t st) {
  if (dtype == Bf16::id) {
    if (D == 64) return launch_pool_t<Bf16, 64>(p, st);
    if (D == 96) return launch_pool_t<Bf16, 96>(p, st);
    if (D == 256) return launch_pool_t<Bf16, 256>(p, st);
    if (D == 512) return launch_pool_t<Bf16, 512>(p, st);
    return launch_pool_t<Bf16, 128>(p, st);
  }
  if (D == 64) return launch_pool_t<F16, 64>(p, st);
  if (D == 96) return launch_pool_t<F16, 96>(p, st);
  if (D == 256) return launch_pool_t<F16, 256>(p, st);
  if (D == 512) return launch_pool_t<F16, 512>(p, st);
  return launch_pool_t<F16, 128>(p, st);
}

// Query blocks per scoring workgroup (one 16-row MFMA tile); 0 = key axis
// too long.
int score_rows_for(int n_kb) { return n_kb <= 16384 ? 16 : 0; }

template <typename T, int D, int KPL>
static hipError_t launch_score_t(const ScoreParams& p, hipStream_t st) {
  dim3 grid((p.n_qb + 15) / 16, p.batch * p.n_slots);
  hipLaunchKernelGGL((score_topk_kernel<T, D, KPL>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}

// keys per lane held in registers for the selection: KPL * 64 >= n_kb
template <typename T, int D>
static hipError_t launch_score_d(const ScoreParams& p, hipStream_t st) {
  if (p.n_kb <= 256) return launch_score_t<T, D, 4>(p, st);
  if (p.n_kb <= 512) return launch_score_t<T, D, 8>(p, st);
  if (p.n_kb <= 1024) return launch_score_t<T, D, 16>(p, st);
  if (p.n_kb <= 2048) return launch_score_t<T, D, 32>(p, st);
  return launch_score_t<T, D, 0>(p, st);
}

hipError_t launch_score(const ScoreParams& p, int dtype, int D, hipStream_t st) {
  if (dtype == Bf16::id) {
    if (D == 64) return launch_score_d<Bf16, 64>(p, st);
    if (D == 96) return launch_score_d<Bf16, 96>(p, st);
    if (D == 256) return launch_score_d<Bf16, 256>(p, st);
    if (D == 512) return launch_score_d<Bf16, 512>(p, st);
    return launch_score_d<Bf16, 128>(p, st);
  }
  if (D == 64) return launch_score_d<F16, 64>(p, st);
  if (D == 96) return launch_score_d<F16, 96>(p, st);
  if (D == 256) return launch_score_d<F16, 256>(p, st);
  if (D == 512) return launch_score_d<F16, 512>(p, st);
  return launch_score_d<F16, 128>(p, st);
}

}  // namespace msa
