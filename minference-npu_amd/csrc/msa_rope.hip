// Rotary position embedding of a layer's query and key heads in one pass.
//
// out[:rot/2]  = r(r(x[:rot/2] * cos[:rot/2]) - r(x[rot/2:rot] * sin[:rot/2]))
// out[rot/2:rot] = r(r(x[rot/2:rot] * cos[rot/2:]) + r(x[:rot/2] * sin[rot/2:]))
// out[rot:]    = x[rot:]
// with r() = round to the input dtype (nearest even) and the sums in fp32:
// the op-by-op rounding of the eager rotate-half form q * cos +
// rotate_half(q) * sin that HF Phi-3 / Llama apply (each elementwise op of a
// 16-bit tensor computes in fp32 and rounds its result), so the output is
// bit-identical to it.
//
// Work item = one 8-element chunk pair (x[c], x[c + rot/2]) or one 8-element
// pass-through chunk of one head row, for each token; query heads come before
// the key heads, which is memory order for the views of a fused qkv
// projection output [B, S, (H + 2 H_kv) D].

#include <algorithm>

#include "msa_kernels.h"

namespace msa {

namespace {

// Round to the 16-bit type (fp16: the hardware conversion, nearest even).
template <typename T>
__device__ inline uint16_t rnd(float f) {
  return T::from_float(f);
}

template <typename T>
__device__ inline float val(uint16_t b) {
  return T::to_float(b);
}

// A block owns kRopeTok consecutive tokens (batch-major) and every head of
// them: the tokens' cos/sin rows are staged in LDS once, each wave takes
// whole head rows (64 / (D / 8) of them; lane l holds 16-byte chunk l of its
// run), and the waves walk the tokens, kRopeUnroll of them with their loads
// in flight.  A load or store instruction therefore covers up to 1 KB of
// contiguous memory for the views of a fused qkv projection; the rotation
// partner of a chunk (x[i +- rot/2]) comes from the lane rot/16 away.
constexpr int kRopeTok = 16;
constexpr int kRopeUnroll = 4;

template <typename T>
__device__ inline u32x4 rope_chunk(const u32x4& x4, const u32x4& p4, const u32x4& c4,
                                   const u32x4& s4, bool lo) {
  // Every product is rounded before the sum; without this the compiler may
  // fuse a product into the subtraction or addition (fp16: v_pk_fma_f16) and
  // skip that rounding.
#pragma clang fp contract(off)
  const uint16_t* x = reinterpret_cast<const uint16_t*>(&x4);
  const uint16_t* p = reinterpret_cast<const uint16_t*>(&p4);
  const uint16_t* c = reinterpret_cast<const uint16_t*>(&c4);
  const uint16_t* sn = reinterpret_cast<const uint16_t*>(&s4);
  u32x4 o4;
  uint16_t* o = reinterpret_cast<uint16_t*>(&o4);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = val<T>(rnd<T>(val<T>(x[i]) * val<T>(c[i])));
    const float b = val<T>(rnd<T>(val<T>(p[i]) * val<T>(sn[i])));
    o[i] = rnd<T>(lo ? a - b : a + b);
  }
  return o4;
}

// bf16: fp32 products and sums rounded by the hardware pack conversion
// (v_cvt_pk_bf16_f32, round to nearest even), two values per instruction;
// a bf16 word widens to fp32 by a shift (low half) or a mask (high half).
// The rotate-half sign is applied as a sign flip of the rounded second
// product, which is what rounding (-x2) * sin gives.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ inline uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
__device__ inline float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <>
__device__ inline u32x4 rope_chunk<Bf16>(const u32x4& x4, const u32x4& p4, const u32x4& c4,
                                         const u32x4& s4, bool lo) {
#pragma clang fp contract(off)
  const uint32_t flip = lo ? 0x80000000u : 0u;
  u32x4 o4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t a = pack_bf16(lo_f(x4[i]) * lo_f(c4[i]), hi_f(x4[i]) * hi_f(c4[i]));
    const uint32_t b = pack_bf16(lo_f(p4[i]) * lo_f(s4[i]), hi_f(p4[i]) * hi_f(s4[i]));
    const float b0 = __uint_as_float(__float_as_uint(lo_f(b)) ^ flip);
    const float b1 = __uint_as_float(__float_as_uint(hi_f(b)) ^ flip);
    o4[i] = pack_bf16(lo_f(a) + b0, hi_f(a) + b1);
  }
  return o4;
}

__device__ inline u32x4 from_lane(const u32x4& v, int src_lane) {
  u32x4 r;
  r.x = __builtin_amdgcn_ds_bpermute(src_lane << 2, int(v.x));
  r.y = __builtin_amdgcn_ds_bpermute(src_lane << 2, int(v.y));
  r.z = __builtin_amdgcn_ds_bpermute(src_lane << 2, int(v.z));
  r.w = __builtin_amdgcn_ds_bpermute(src_lane << 2, int(v.w));
  return r;
}

template <typename T>
__global__ __launch_bounds__(1024) void rope_kernel(const RopeParams P) {
  __shared__ __attribute__((aligned(16))) uint16_t tab[kRopeTok * 2 * kRopeMaxRot];
  const int64_t n_all = int64_t(P.batch) * P.s;
  const int64_t tok0 = int64_t(blockIdx.x) * kRopeTok;
  const int n_tok = int(min(int64_t(kRopeTok), n_all - tok0));
  const int b0 = int(tok0 / P.s);
  const int s0 = int(tok0 - int64_t(b0) * P.s);
  const int rc = P.rot / 8;  // 16-byte chunks per table row

  // cos/sin rows of this block's tokens -> LDS [token][table][rot]
  for (int i = threadIdx.x; i < n_tok * 2 * rc; i += blockDim.x) {
    const int t = i / (2 * rc);
    const int r = i - t * 2 * rc;
    const int tb = r / rc;
    const int c = r - tb * rc;
    int b = b0, s = s0 + t;
    while (s >= P.s) { s -= P.s; ++b; }
    const uint16_t* src = tb ? static_cast<const uint16_t*>(P.sin) + b * P.n_sb + s * P.n_ss
                             : static_cast<const uint16_t*>(P.cos) + b * P.c_sb + s * P.c_ss;
    *reinterpret_cast<u32x4*>(tab + (t * 2 + tb) * P.rot + 8 * c) = load16(src + 8 * c);
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int cpr = P.n_pair * 2 + P.n_pass;  // 16-byte chunks per head row (D / 8)
  const int hpw = 64 / cpr;                 // head rows per wave
  const int hl = lane / cpr;
  const int j = lane - hl * cpr;             // chunk of the row
  const int half_c = P.n_pair;               // rot / 16: partner distance in lanes
  const bool rotated = j < 2 * half_c;
  const bool lo = j < half_c;
  const int partner = rotated ? (lo ? lane + half_c : lane - half_c) : lane;
  const int n_heads = P.heads + P.kv_heads;
  const int n_groups = (n_heads + hpw - 1) / hpw;
  const int n_waves = blockDim.x >> 6;
  for (int g = threadIdx.x >> 6; g < n_groups; g += n_waves) {
    const int head = g * hpw + hl;
    const bool active = hl < hpw && head < n_heads;  // uniform per lane group
    const bool is_q = head < P.heads;
    const int h = is_q ? head : head - P.heads;
    const uint16_t* xbase = static_cast<const uint16_t*>(is_q ? P.q : P.k) +
                            (is_q ? h * P.q_sh : h * P.k_sh) + 8 * j;
    uint16_t* ybase = static_cast<uint16_t*>(is_q ? P.qo : P.ko) +
                      (is_q ? h * P.qo_sh : h * P.ko_sh) + 8 * j;
    const int64_t xsb = is_q ? P.q_sb : P.k_sb, xss = is_q ? P.q_ss : P.k_ss;
    const int64_t ysb = is_q ? P.qo_sb : P.ko_sb, yss = is_q ? P.qo_ss : P.ko_ss;
    int b = b0, s = s0;
    for (int t0 = 0; t0 < n_tok; t0 += kRopeUnroll) {
      uint16_t* yp[kRopeUnroll];
      u32x4 x[kRopeUnroll];
#pragma unroll
      for (int u = 0; u < kRopeUnroll; ++u) {
        yp[u] = ybase + b * ysb + s * yss;
        x[u] = zero_u32x4();
        if (active && t0 + u < n_tok) x[u] = load16(xbase + b * xsb + s * xss);
        if (++s == P.s) { s = 0; ++b; }
      }
#pragma unroll
      for (int u = 0; u < kRopeUnroll; ++u) {
        if (t0 + u >= n_tok) break;  // uniform across the block
        const u32x4 px = from_lane(x[u], partner);  // every lane takes part
        if (!active) continue;
        u32x4 o = x[u];
        if (rotated) {
          const uint16_t* cs = tab + ((t0 + u) * 2) * P.rot + 8 * j;
          const u32x4 c4 = *reinterpret_cast<const u32x4*>(cs);
          const u32x4 s4 = *reinterpret_cast<const u32x4*>(cs + P.rot);
          o = rope_chunk<T>(x[u], px, c4, s4, lo);
        }
        store16(yp[u], o);
      }
    }
  }
}

}  // namespace

hipError_t launch_rope(const RopeParams& p, int dtype, hipStream_t st) {
  const int64_t n_tok = int64_t(p.batch) * p.s;
  const dim3 grid(uint32_t((n_tok + kRopeTok - 1) / kRopeTok));
  const int hpw = 64 / (2 * p.n_pair + p.n_pass);
  const int n_groups = (p.heads + p.kv_heads + hpw - 1) / hpw;
  const dim3 block(uint32_t(64 * std::min(16, n_groups)));
  if (dtype == Bf16::id)
    hipLaunchKernelGGL(rope_kernel<Bf16>, grid, block, 0, st, p);
  else
    hipLaunchKernelGGL(rope_kernel<F16>, grid, block, 0, st, p);
  return hipGetLastError();
}

}  // namespace msa
