// Shared device helpers for the MI355X (gfx950) sparse prefill attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace msa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlock = 64;      // token block == q tile == k tile
constexpr int kMaxHeads = 128;  // head descriptors carried in the kernel arguments

// Element tags for the 16-bit input types.
struct Bf16 {
  static constexpr int id = 1;
  __device__ static float to_float(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
  // Round-to-nearest-even fp32 -> bf16 (finite inputs).
  __device__ static uint16_t from_float(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u) return uint16_t(u >> 16);  // inf/nan pass through
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
  }
};

struct F16 {
  static constexpr int id = 2;
  __device__ static float to_float(uint16_t b) {
    return float(__builtin_bit_cast(_Float16, b));
  }
  __device__ static uint16_t from_float(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
};

// fp32 to fp16 after multiplying by sc (a power of two): finite values
// saturate at the fp16 finite range, Inf and NaN pass through unchanged.
__device__ inline _Float16 to_f16_scaled(float f, float sc) {
  f *= sc;
  f = __builtin_isfinite(f) ? fminf(fmaxf(f, -65504.0f), 65504.0f) : f;
  return static_cast<_Float16>(f);
}

// |f| for finite f, 0 for Inf / NaN (the magnitude a scale must bring into
// fp16 range; non-finite values keep their meaning at any scale).
__device__ inline float finite_abs(float f) { return __builtin_isfinite(f) ? fabsf(f) : 0.0f; }

// Largest finite fp16 magnitude.
constexpr float kF16Max = 65504.0f;

__device__ inline u32x4 zero_u32x4() { return u32x4{0u, 0u, 0u, 0u}; }

// Load of read-only data at a wave-uniform address through the constant
// address space, which the compiler lowers to a scalar load.  For data a
// kernel never writes (tile lists, counts, masks written by earlier
// launches).  A vector load would land in a VGPR behind the wave's
// outstanding operand loads: its wait, which counts vector loads in order,
// would also wait for every operand load issued before it.
template <typename T>
__device__ inline T load_uniform(const T* p) {
  return *reinterpret_cast<const __attribute__((address_space(4))) T*>(
      __builtin_bit_cast(uintptr_t, p));
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16x16x32 MFMA on 16-bit inputs, fp32 accumulation.  Lane l: A[l % 16][8 (l / 16) + j],
// B[8 (l / 16) + j][l % 16], C[4 (l / 16) + i][l % 16].
template <typename T>
__device__ inline f32x4 mfma_qk(u32x4 a, u32x4 b, f32x4 c);

template <>
__device__ inline f32x4 mfma_qk<Bf16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <>
__device__ inline f32x4 mfma_qk<F16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

__device__ inline u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ inline void store16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

}  // namespace msa
