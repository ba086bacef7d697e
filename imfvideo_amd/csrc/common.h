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

// An fp32 result held as such before a 16-bit conversion.  (x * y).to(f16)
// rounds the fp32 product and then the 16-bit value; left alone, the compiler
// fuses a multiply (or fma) and the conversion into one rounding
// (v_fma_mix*_f16), which differs where the fp32 result lands on a 16-bit
// rounding midpoint.  Every fp16 conversion here goes through it (bf16 has no
// fused form).
__device__ inline float keep_f32(float x) {
  asm("" : "+v"(x));
  return x;
}

// 16-bit storage tags.  Values travel as raw uint16 bits; `to_f32` widens
// exactly, `from_f32` rounds to nearest even (hardware cvt on gfx950).
struct F16 {
  static constexpr int kDtype = SLA2H_DTYPE_F16;
  __device__ static inline float to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
  }
  __device__ static inline uint16_t from_f32(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)keep_f32(f));
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

typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

// Two fp32 -> one packed pair of 16-bit values (round to nearest even),
// a single v_cvt_pk_* instruction.
template <typename T16>
__device__ inline uint32_t pack_pair(float lo, float hi);
template <>
__device__ inline uint32_t pack_pair<BF16>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
}
template <>
__device__ inline uint32_t pack_pair<F16>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_convertvector((f32x2{keep_f32(lo), keep_f32(hi)}), f16x2));
}

// Reductions over the four 16-lane rows of a wave64 (lanes l, l^16, l^32,
// l^48) with the gfx950 row-swap permutes: VALU only, no LDS round trip.
// permlane16_swap(x, x) yields (x[l & ~16], x[l | 16]) and
// permlane32_swap(x, x) yields (x[l & ~32], x[l | 32]).
__device__ inline float2 swap16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  return make_float2(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ inline float2 swap32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                  __builtin_bit_cast(unsigned, v), false, false);
  return make_float2(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ inline float max_over_groups(float v) {
  float2 a = swap16(v);
  v = fmaxf(a.x, a.y);
  a = swap32(v);
  return fmaxf(a.x, a.y);
}
// (x0 + x1) + (x2 + x3) with the row pairs in a fixed order: every lane of a
// column gets the bit-identical sum.
__device__ inline float sum_over_groups(float v) {
  float2 a = swap16(v);
  v = a.x + a.y;
  a = swap32(v);
  return a.x + a.y;
}

// Raw buffer resources (gfx9 descriptor, stride 0, byte-addressed): loads
// past num_bytes return zeros, and offsets are 32-bit VGPRs.
// `base` and `num_bytes` must be wave-uniform; they are pinned to SGPRs here
// (64-bit products may be computed on the VALU, and a VGPR descriptor would
// make every load a readfirstlane waterfall loop).
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t num_bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  void* p = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, 0, __builtin_amdgcn_readfirstlane((int)num_bytes),
                                           0x00020000);
}
__device__ inline u32x4 buf_load16(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0));
}
__device__ inline u32x2 buf_load8(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, 0));
}

// 2^x on the hardware exp unit (v_exp_f32); inputs here are <= 0 or -inf.
__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Ascending sort of the n tile ids of a visiting list in LDS (element i read
// with get(i), written with set(i, id)).  Workgroups that visit their tiles in
// ascending order sweep the key tiles of a head together and share them in
// the XCD's L2.  Up to 64 ids: a bitonic sort in the registers of wave 0
// (threads 0..63); more: rank by counting into tmp (n ints of LDS), ties by
// position.  Called by every thread of a 256-thread workgroup after the list
// is complete in LDS (barrier included); ends with a barrier.
template <typename Get, typename Set>
__device__ inline void sort_ids_ascending(int n, int tid, Get get, Set set, int* tmp) {
  if (n <= 64) {
    if (tid < 64) {
      int v = tid < n ? get(tid) : 0x7fffffff;
#pragma unroll
      for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (int jj = k >> 1; jj > 0; jj >>= 1) {
          const int o = __shfl_xor(v, jj);
          v = (((tid & jj) == 0) == ((tid & k) == 0)) ? min(v, o) : max(v, o);
        }
      }
      if (tid < n) set(tid, v);
    }
  } else {
    for (int j = tid; j < n; j += 256) {
      const int nj = get(j);
      int c = 0;
      for (int i = 0; i < n; ++i) {
        const int ni = get(i);
        c += (ni < nj) || (ni == nj && i < j);
      }
      tmp[c] = nj;
    }
    __syncthreads();
    for (int j = tid; j < n; j += 256) set(j, tmp[j]);
  }
  __syncthreads();
}

}  // namespace sla2h

#define SLA2H_CHECK_ARG(cond) \
  do {                        \
    if (!(cond)) return (int)hipErrorInvalidValue; \
  } while (0)
