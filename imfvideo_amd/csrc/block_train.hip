// Fused elementwise stages of the DiT block's training forward / backward
// (autograd path), gfx950.  HBM-bound: each element is read and written once,
// fp32 arithmetic, 16-bit or fp32 I/O, 16 bytes per thread access.
//
//   situ_mul_fwd   h = situ(g) u',  situ(g) = beta tanh(g / beta) sigmoid(g),
//                  u' = lb tanh(u / lb) with a soft clamp lb > 0, else u
//   situ_mul_bwd   dg = dh u' situ'(g),  du = dh situ(g) du'/du,
//                  situ'(g) = (1 - tanh^2(g / beta)) sigmoid(g)
//                             + beta tanh(g / beta) sigmoid(g) (1 - sigmoid(g)),
//                  du'/du = 1 - tanh^2(u / lb) (1 without the clamp)
//
// Reference semantics: models/imf_dit_video.py:136-171 (SituAndMul.forward,
// evaluated in fp32 from the input dtype and cast back; its backward is torch
// autograd of that fp32 expression).
#include "common.h"

#include <initializer_list>
#include <type_traits>
#include <utility>

namespace sla2h {

namespace {

constexpr int kF32 = 2;  // dtype code of fp32 I/O (SLA2H_DTYPE_F16 = 0, SLA2H_DTYPE_BF16 = 1)

// VEC consecutive elements <-> fp32 (VEC = 8 for 16-bit, 4 for fp32: 16 bytes)
template <int DT>
struct Vec;
template <>
struct Vec<kF32> {
  static constexpr int N = 4;
  __device__ static void ld(const void* p, int64_t i, float (&x)[N]) {
    const float4 v = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    x[0] = v.x, x[1] = v.y, x[2] = v.z, x[3] = v.w;
  }
  __device__ static void st(void* p, int64_t i, const float (&x)[N]) {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(x[0], x[1], x[2], x[3]);
  }
};
template <typename T16>
struct Vec16 {
  static constexpr int N = 8;
  __device__ static void ld(const void* p, int64_t i, float (&x)[N]) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p) + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = T16::to_f32((uint16_t)(v[e] & 0xffff));
      x[2 * e + 1] = T16::to_f32((uint16_t)(v[e] >> 16));
    }
  }
  __device__ static void st(void* p, int64_t i, const float (&x)[N]) {
    u32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = pack_pair<T16>(x[2 * e], x[2 * e + 1]);
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p) + i) = v;
  }
};
template <>
struct Vec<SLA2H_DTYPE_F16> : Vec16<F16> {};
template <>
struct Vec<SLA2H_DTYPE_BF16> : Vec16<BF16> {};

// one element per thread (shapes or strides that do not allow 16-byte accesses)
template <int DT>
struct Vec1 {
  static constexpr int N = 1;
  __device__ static void ld(const void* p, int64_t i, float (&x)[N]) {
    if (DT == kF32)
      x[0] = static_cast<const float*>(p)[i];
    else if (DT == SLA2H_DTYPE_BF16)
      x[0] = BF16::to_f32(static_cast<const uint16_t*>(p)[i]);
    else
      x[0] = F16::to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  __device__ static void st(void* p, int64_t i, const float (&x)[N]) {
    if (DT == kF32)
      static_cast<float*>(p)[i] = x[0];
    else if (DT == SLA2H_DTYPE_BF16)
      static_cast<uint16_t*>(p)[i] = BF16::from_f32(x[0]);
    else
      static_cast<uint16_t*>(p)[i] = F16::from_f32(x[0]);
  }
};
template <int DT, bool WIDE>
using VecOf = typename std::conditional<WIDE, Vec<DT>, Vec1<DT>>::type;

__device__ inline float sigmoid_f(float x) { return 1.f / (1.f + __expf(-x)); }

template <int DT, bool WIDE>
__global__ __launch_bounds__(256) void situ_mul_fwd_kernel(const void* __restrict__ G,
                                                           const void* __restrict__ U,
                                                           int64_t rows, int F, int64_t sg,
                                                           int64_t su, float beta, float lb,
                                                           void* __restrict__ OUT) {
  using V = VecOf<DT, WIDE>;
  constexpr int N = V::N;
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * N;
  if (idx >= rows * F) return;
  const int64_t row = idx / F;
  const int c = (int)(idx - row * F);
  float g[N], u[N], h[N];
  V::ld(G, row * sg + c, g);
  V::ld(U, row * su + c, u);
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float act = beta * tanhf(g[e] / beta) * sigmoid_f(g[e]);
    const float uc = lb > 0.f ? lb * tanhf(u[e] / lb) : u[e];
    h[e] = act * uc;
  }
  V::st(OUT, idx, h);
}

template <int DT, bool WIDE>
__global__ __launch_bounds__(256) void situ_mul_bwd_kernel(const void* __restrict__ DH,
                                                           const void* __restrict__ G,
                                                           const void* __restrict__ U,
                                                           int64_t rows, int F, int64_t sg,
                                                           int64_t su, float beta, float lb,
                                                           void* __restrict__ DG,
                                                           void* __restrict__ DU) {
  using V = VecOf<DT, WIDE>;
  constexpr int N = V::N;
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * N;
  if (idx >= rows * F) return;
  const int64_t row = idx / F;
  const int c = (int)(idx - row * F);
  float dh[N], g[N], u[N], dg[N], du[N];
  V::ld(DH, idx, dh);
  V::ld(G, row * sg + c, g);
  V::ld(U, row * su + c, u);
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float th = tanhf(g[e] / beta);
    const float sg_ = sigmoid_f(g[e]);
    const float act = beta * th * sg_;
    const float dact = (1.f - th * th) * sg_ + beta * th * sg_ * (1.f - sg_);
    float uc = u[e], duc = 1.f;
    if (lb > 0.f) {
      const float tu = tanhf(u[e] / lb);
      uc = lb * tu;
      duc = 1.f - tu * tu;
    }
    dg[e] = dh[e] * uc * dact;
    du[e] = dh[e] * act * duc;
  }
  V::st(DG, idx, dg);
  V::st(DU, idx, du);
}

template <int DT>
bool wide_ok(int F, std::initializer_list<std::pair<const void*, int64_t>> ps) {
  constexpr int N = Vec<DT>::N;
  if (F % N) return false;
  for (const auto& p : ps)
    if (reinterpret_cast<uintptr_t>(p.first) % 16 || p.second % N) return false;
  return true;
}

}  // namespace

}  // namespace sla2h

using namespace sla2h;

// grid of `threads` 256-thread blocks, or 0 when it does not fit
static unsigned grid_of(int64_t threads) {
  const int64_t g = (threads + 255) / 256;
  return g < (1ll << 31) ? (unsigned)g : 0u;
}

extern "C" int sla2h_situ_mul_fwd(const void* gate, const void* up, int dtype, int64_t rows,
                                  int F, int64_t sg, int64_t su, float beta, float lb, void* out,
                                  void* stream) {
  SLA2H_CHECK_ARG(gate && up && out);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16 || dtype == kF32);
  SLA2H_CHECK_ARG(rows > 0 && F > 0 && sg >= F && su >= F && beta > 0.f && lb >= 0.f);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto go = [&](auto dt) -> int {
    constexpr int DT = decltype(dt)::value;
    const bool wide = wide_ok<DT>(F, {{gate, sg}, {up, su}, {out, F}});
    const unsigned grid = grid_of(rows * F / (wide ? Vec<DT>::N : 1));
    if (grid == 0) return (int)hipErrorInvalidValue;
    if (wide)
      situ_mul_fwd_kernel<DT, true><<<grid, 256, 0, st>>>(gate, up, rows, F, sg, su, beta, lb, out);
    else
      situ_mul_fwd_kernel<DT, false><<<grid, 256, 0, st>>>(gate, up, rows, F, sg, su, beta, lb, out);
    return (int)hipGetLastError();
  };
  if (dtype == SLA2H_DTYPE_BF16) return go(std::integral_constant<int, SLA2H_DTYPE_BF16>{});
  if (dtype == SLA2H_DTYPE_F16) return go(std::integral_constant<int, SLA2H_DTYPE_F16>{});
  return go(std::integral_constant<int, kF32>{});
}

extern "C" int sla2h_situ_mul_bwd(const void* dh, const void* gate, const void* up, int dtype,
                                  int64_t rows, int F, int64_t sg, int64_t su, float beta,
                                  float lb, void* dgate, void* dup, void* stream) {
  SLA2H_CHECK_ARG(dh && gate && up && dgate && dup);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16 || dtype == kF32);
  SLA2H_CHECK_ARG(rows > 0 && F > 0 && sg >= F && su >= F && beta > 0.f && lb >= 0.f);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto go = [&](auto dt) -> int {
    constexpr int DT = decltype(dt)::value;
    const bool wide = wide_ok<DT>(F, {{gate, sg}, {up, su}, {dh, F}, {dgate, F}, {dup, F}});
    const unsigned grid = grid_of(rows * F / (wide ? Vec<DT>::N : 1));
    if (grid == 0) return (int)hipErrorInvalidValue;
    if (wide)
      situ_mul_bwd_kernel<DT, true><<<grid, 256, 0, st>>>(dh, gate, up, rows, F, sg, su, beta, lb,
                                                          dgate, dup);
    else
      situ_mul_bwd_kernel<DT, false><<<grid, 256, 0, st>>>(dh, gate, up, rows, F, sg, su, beta, lb,
                                                           dgate, dup);
    return (int)hipGetLastError();
  };
  if (dtype == SLA2H_DTYPE_BF16) return go(std::integral_constant<int, SLA2H_DTYPE_BF16>{});
  if (dtype == SLA2H_DTYPE_F16) return go(std::integral_constant<int, SLA2H_DTYPE_F16>{});
  return go(std::integral_constant<int, kF32>{});
}
