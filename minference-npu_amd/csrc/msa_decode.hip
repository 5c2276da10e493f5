// Decode attention: one query row per head against the whole KV cache.
//
// Reference semantics: decode_dense, MInference-NPU/minference/backend_npu/attention.py:274-314
// (q [B,H,1,D], k/v cache [B,H_kv,S,D], scale default 1/sqrt(D), every key
// visible), dispatched for q_len == 1 by
// MInference-NPU/minference/modules/minference_forward.py:488-490.
//
// The work is a GEMV pair per head and is bound by HBM (K and V are read
// once, 4*D bytes per key); MFMA would waste 15 of 16 rows, so it runs on
// the VALU in fp32.
//
// Split-K: the grid is (n_split, B*H); workgroup (s, b*H+h) walks keys
// [s*chunk, min((s+1)*chunk, S)) of head h in 16-key blocks, wave w taking
// blocks w, w+4, ...  A block of K is 16 rows of D elements; with rows
// contiguous it is 16*D*2 bytes read as D/32 one-kilobyte loads per wave
// (lane l, load i: elements f = 8l + 512i .. +7 of the block, always inside
// row f / D).  Each lane forms the partial dot products of its 8-element
// pieces, the 16 key dot products reduce through wave-private LDS, the
// online softmax runs on 16 lanes, and P is read back per piece for the PV
// update of the same pieces of V.  Rows with another stride use the same
// pieces, addressed row by row.
//
// Each workgroup leaves O[D] and (m, l) for its key range in the workspace;
// the combine kernel merges the splits of a head and writes the output row.

#include "msa_common.h"
#include "msa_kernels.h"

namespace msa {

template <typename T, int D>
__global__ __launch_bounds__(256) void decode_kernel(DecodeParams P) {
  constexpr int NL = D / 32;   // 1 KB loads per 16-key block of K (and of V)
  constexpr int NPC = D / 8;   // 8-element pieces per key row
  __shared__ float part[4][16][NPC + 1];  // per-wave partial dot products
  __shared__ float pw[4][16];             // per-wave P of the block
  __shared__ float om[4][64 * NL * 8 + 2];  // merge: per-wave O pieces, m, l

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int split = blockIdx.x;
  const int bh = blockIdx.y;  // b * heads + h
  const int b = bh / P.heads;
  const int h = bh - b * P.heads;
  const int kvh = h / P.kv_group;

  const int j_begin = split * P.chunk;
  const int j_end = min(j_begin + P.chunk, P.s_k);

  // this lane's pieces: key row kr_i of the block, first element d0_i
  int key_i[NL], d0_i[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int f = 8 * lane + 512 * i;
    key_i[i] = f / D;
    d0_i[i] = f - key_i[i] * D;
  }
  // q pieces in fp32
  float qv[NL][8];
  {
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(P.q) + b * P.q_sb + int64_t(h) * P.q_sh;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const u32x4 x = load16(qrow + d0_i[i]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qv[i][2 * e] = T::to_float(uint16_t(x[e] & 0xffffu));
        qv[i][2 * e + 1] = T::to_float(uint16_t(x[e] >> 16));
      }
    }
  }

  // Buffer descriptors bounded at row S, so pieces of rows >= S read 0.
  const unsigned char* kbase = reinterpret_cast<const unsigned char*>(P.k) +
                               2 * (b * P.k_sb + int64_t(kvh) * P.k_sh);
  const unsigned char* vbase = reinterpret_cast<const unsigned char*>(P.v) +
                               2 * (b * P.v_sb + int64_t(kvh) * P.v_sh);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<unsigned char*>(kbase), short(0), int(int64_t(P.s_k) * P.k_ss * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<unsigned char*>(vbase), short(0), int(int64_t(P.s_k) * P.v_ss * 2), 0x00020000);
  uint32_t koff[NL], voff[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    koff[i] = uint32_t(key_i[i]) * uint32_t(P.k_ss) * 2u + 2u * d0_i[i];
    voff[i] = uint32_t(key_i[i]) * uint32_t(P.v_ss) * 2u + 2u * d0_i[i];
  }
  // K and V are read once per call: loads carry the non-temporal hint (cache
  // policy bit 1) so the stream does not evict reused lines.
  auto load_block = [&](int j0, u32x4 (&kr)[NL], u32x4 (&vr)[NL]) __attribute__((always_inline)) {
    const int ks = j0 * int(P.k_ss) * 2, vs = j0 * int(P.v_ss) * 2;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      kr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, koff[i], ks, 2));
      vr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, voff[i], vs, 2));
    }
  };

  float o[NL][8];
#pragma unroll
  for (int i = 0; i < NL; ++i)
#pragma unroll
    for (int u = 0; u < 8; ++u) o[i][u] = 0.0f;
  float m = -__builtin_inff();  // running max (scaled, log2 units), wave-uniform
  float l = 0.0f;               // running sum (lanes 0..15 hold partial sums)
  const float c = P.scale_log2;

  // one 16-key block: scores, online softmax, O update
  auto block = [&](int j0, const u32x4(&kc)[NL], const u32x4(&vc)[NL]) __attribute__((always_inline)) {
    // partial dot products of this lane's pieces
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc = __builtin_fmaf(qv[i][2 * e], T::to_float(uint16_t(kc[i][e] & 0xffffu)), acc);
        acc = __builtin_fmaf(qv[i][2 * e + 1], T::to_float(uint16_t(kc[i][e] >> 16)), acc);
      }
      part[w][key_i[i]][d0_i[i] / 8] = acc;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    // lanes 0..15: the block's 16 scores
    float s = -__builtin_inff();
    if (lane < 16) {
      float acc = 0.0f;
#pragma unroll
      for (int p = 0; p < NPC; ++p) acc += part[w][lane][p];
      s = (j0 + lane < j_end) ? acc * c : -__builtin_inff();
    }
    float bm = s;
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) bm = fmaxf(bm, __shfl_xor(bm, off, 64));
    bm = __shfl(bm, 0, 64);
    const float mn = fmaxf(m, bm);
    const float alpha = __builtin_amdgcn_exp2f(m - mn);  // m = -inf at first: exp2(-inf) = 0
    m = mn;
    const float p = lane < 16 ? __builtin_amdgcn_exp2f(s - m) : 0.0f;
    l = l * alpha + p;
    if (lane < 16) pw[w][lane] = p;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const float pi = pw[w][key_i[i]];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[i][2 * e] = __builtin_fmaf(pi, T::to_float(uint16_t(vc[i][e] & 0xffffu)), o[i][2 * e] * alpha);
        o[i][2 * e + 1] = __builtin_fmaf(pi, T::to_float(uint16_t(vc[i][e] >> 16)), o[i][2 * e + 1] * alpha);
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // Wave w takes blocks first + 64 i, i < nblk, two blocks in flight ahead
  // of the one being reduced, in three rotating register sets.  Loads past
  // the wave's last block repeat that block, so every load is unconditional
  // and in range.
  const int first = j_begin + 16 * w;
  const int nblk = j_end > first ? (j_end - first + 63) / 64 : 0;
  const int last = first + 64 * max(nblk - 1, 0);
  auto jb = [&](int i) { return min(first + 64 * i, last); };
  u32x4 ka[NL], va[NL], kb[NL], vb[NL], kc[NL], vc[NL];
  load_block(jb(0), ka, va);
  load_block(jb(1), kb, vb);
  for (int i = 0; i < nblk; i += 3) {
    load_block(jb(i + 2), kc, vc);
    block(first + 64 * i, ka, va);
    if (i + 1 >= nblk) break;
    load_block(jb(i + 3), ka, va);
    block(first + 64 * (i + 1), kb, vb);
    if (i + 2 >= nblk) break;
    load_block(jb(i + 4), kb, vb);
    block(first + 64 * (i + 2), kc, vc);
  }

  // ---- merge the 4 waves and the 16 key positions of every piece
  // wave sum of l over lanes 0..15
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) l += __shfl_xor(l, off, 64);
  float* mine = om[w];
#pragma unroll
  for (int i = 0; i < NL; ++i)
#pragma unroll
    for (int u = 0; u < 8; ++u) mine[(64 * i + lane) * 8 + u] = o[i][u];
  if (lane == 0) {
    mine[64 * NL * 8] = m;
    mine[64 * NL * 8 + 1] = l;
  }
  __syncthreads();
  // elements d = t, t + 256, ... of O (thread t), summing every (wave,
  // piece) whose piece covers d, each wave scaled by exp2(m_w - M)
  for (int d = tid; d < D; d += 256) {
    float mw[4], M = -__builtin_inff();
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      mw[v] = om[v][64 * NL * 8];
      M = fmaxf(M, mw[v]);
    }
    float L = 0.0f, acc = 0.0f;
    const int dp = d & ~7, du = d & 7;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float f = M == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(mw[v] - M);
      L += f * om[v][64 * NL * 8 + 1];
      float sv = 0.0f;
      for (int r = 0; r < 16; ++r) {  // piece of key row r covering d
        const int fl = r * D + dp;    // flat element of that piece in the block
        const int i = fl / 512, ln = (fl - 512 * i) / 8;
        sv += om[v][(64 * i + ln) * 8 + du];
      }
      acc += f * sv;
    }
    const int64_t row = int64_t(bh) * P.n_split + split;
    P.part[row * D + d] = acc;
    if (d == 0) {
      P.ml[2 * row] = M;
      P.ml[2 * row + 1] = L;
    }
  }
}

// Merge the splits of one head: O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s.
// Every load is independent: the (m, l) pairs are read once into LDS, then
// G groups of D/4 threads each sum a stride of splits with 16-byte loads and
// the groups reduce through LDS.
template <typename T, bool OUT_F32, int D>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeParams P) {
  constexpr int TPR = D / 4;    // threads per split row, 4 elements each
  constexpr int G = 256 / TPR;  // split groups
  __shared__ float fs[kDecodeMaxSplit];
  __shared__ float red[8];
  __shared__ __align__(16) float acc_g[G][D];
  const int bh = blockIdx.x;
  const int b = bh / P.heads, h = bh - b * P.heads;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int ns = P.n_split;
  const float* ml = P.ml + int64_t(bh) * ns * 2;

  float mx = -__builtin_inff();
  for (int s = tid; s < ns; s += 256) {
    const float ms = ml[2 * s];
    fs[s] = ms;
    mx = fmaxf(mx, ms);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) red[w] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float L = 0.0f;
  for (int s = tid; s < ns; s += 256) {
    const float f = M == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(fs[s] - M);
    fs[s] = f;
    L += f * ml[2 * s + 1];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off, 64);
  if (lane == 0) red[4 + w] = L;
  __syncthreads();
  L = (red[4] + red[5]) + (red[6] + red[7]);

  const int g = tid / TPR, c = tid - g * TPR;
  if (g < G) {
    const float* src = P.part + int64_t(bh) * ns * D + 4 * c;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll 4
    for (int s = g; s < ns; s += G) {
      const float4 x = *reinterpret_cast<const float4*>(src + int64_t(s) * D);
      const float f = fs[s];
      a0 = __builtin_fmaf(f, x.x, a0);
      a1 = __builtin_fmaf(f, x.y, a1);
      a2 = __builtin_fmaf(f, x.z, a2);
      a3 = __builtin_fmaf(f, x.w, a3);
    }
    *reinterpret_cast<float4*>(&acc_g[g][4 * c]) = float4{a0, a1, a2, a3};
  }
  __syncthreads();
  for (int d = tid; d < D; d += 256) {
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < G; ++q) acc += acc_g[q][d];
    const float r = L > 0.0f ? acc / L : 0.0f;
    const int64_t off = b * P.o_sb + int64_t(h) * P.o_sh + d;
    if constexpr (OUT_F32) {
      reinterpret_cast<float*>(P.o)[off] = r;
    } else {
      reinterpret_cast<uint16_t*>(P.o)[off] = T::from_float(r);
    }
  }
}

template <typename T, bool OUT_F32, int D>
static hipError_t launch_decode_t(const DecodeParams& p, hipStream_t st) {
  hipLaunchKernelGGL((decode_kernel<T, D>), dim3(p.n_split, p.batch * p.heads), dim3(256), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((decode_combine_kernel<T, OUT_F32, D>), dim3(p.batch * p.heads), dim3(256), 0,
                     st, p);
  return hipGetLastError();
}

template <typename T, bool OUT_F32>
static hipError_t launch_decode_d(const DecodeParams& p, int D, hipStream_t st) {
  if (D == 64) return launch_decode_t<T, OUT_F32, 64>(p, st);
  if (D == 96) return launch_decode_t<T, OUT_F32, 96>(p, st);
  if (D == 256) return launch_decode_t<T, OUT_F32, 256>(p, st);
  if (D == 512) return launch_decode_t<T, OUT_F32, 512>(p, st);
  return launch_decode_t<T, OUT_F32, 128>(p, st);
}

hipError_t launch_decode(const DecodeParams& p, int dtype, int out_dtype, int D, hipStream_t st) {
  const bool f32 = out_dtype == 3;
  if (dtype == Bf16::id)
    return f32 ? launch_decode_d<Bf16, true>(p, D, st) : launch_decode_d<Bf16, false>(p, D, st);
  return f32 ? launch_decode_d<F16, true>(p, D, st) : launch_decode_d<F16, false>(p, D, st);
}

}  // namespace msa
