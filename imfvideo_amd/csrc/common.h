// Shared device helpers for the gfx950 SLA2 kernels: 16-bit storage types,
// MFMA operand vectors, wave64 reductions and the argument-check macro.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sla2h.h"

namespace sla2h {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) int i32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

// 16-bit storage tags.  Values travel as raw uint16 bits; `to_f32` widens
// exactly, `from_f32` rounds to nearest even (hardware cvt on gfx950).
struct F16 {
  static constexpr int kDtype = SLA2H_DTYPE_F16;
  __device__ static inline float to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
  }
  __device__ static inline uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
};
struct BF16 {
  static constexpr int kDtype = SLA2H_DTYPE_BF16;
  __device__ static inline float to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
  }
  __device__ static inline uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
  }
};

__device__ inline uint16_t bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ inline float bf16_val(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// ---- MFMA wrappers (gfx950).  Operand slot convention used everywhere:
// for a 16x16 output tile, lane l supplies A row (l % 16) and B column (l % 16);
// its K slots are the lane-group g = l / 16 block of the K extent, identical
// for A and B, so any consistent K relabelling gives the same product.
// Output: lane l holds D[4*(l/16) + i][l % 16], i = 0..3.

// 16x16x32, 16-bit operands given as 4 packed uint32 (8 halves).
template <typename T16>
__device__ inline f32x4 mfma_16x16x32(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ inline f32x4 mfma_16x16x32<BF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ inline f32x4 mfma_16x16x32<F16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// 16x16x16, 16-bit operands given as 2 packed uint32 (4 halves).
template <typename T16>
__device__ inline f32x4 mfma_16x16x16(u32x2 a, u32x2 b, f32x4 c);
template <>
__device__ inline f32x4 mfma_16x16x16<BF16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                   __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}
template <>
__device__ inline f32x4 mfma_16x16x16<F16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                               __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
}

// int8 16x16x64: 16 int8 per lane per operand, int32 accumulate.
__device__ inline i32x4 mfma_i8_16x16x64(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// bf16 MFMA on bf16 bit patterns (used for hi/lo split fp32 products).
__device__ inline f32x4 mfma_bf16_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ inline uint32_t pack2(uint16_t lo, uint16_t hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

// xor-shuffle within the wave64 (ds_bpermute).
__device__ inline float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }

__device__ inline float max_over_groups(float v) {  // over lanes l, l^16, l^32, l^48
  v = fmaxf(v, shfl_xor(v, 16));
  v = fmaxf(v, shfl_xor(v, 32));
  return v;
}
__device__ inline float sum_over_groups(float v) {
  v += shfl_xor(v, 16);
  v += shfl_xor(v, 32);
  return v;
}

}  // namespace sla2h

#define SLA2H_CHECK_ARG(cond) \
  do {                        \
    if (!(cond)) return (int)hipErrorInvalidValue; \
  } while (0)
