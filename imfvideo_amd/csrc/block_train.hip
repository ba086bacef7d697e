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

// ---------------------------------------------------------------------------
// RMSNorm of the training forward and its backward (models/imf_dit_video.py:
// 121-133): y = round_x(x r) w with r = 1 / sqrt(mean(x^2) + eps) in fp32,
// round_x the rounding to x's dtype, w fp32, y fp32 (the product promotes).
// Backward (autograd of that expression): g = round_x(dy w) (the gradient of
// the cast is taken in x's dtype), dx = round_x(r g - x r^3 mean(g x)),
// dw = sum over rows of round_x(x r) dy.  One wave per row, each lane a
// strided set of the row's D <= 1024 channels; dw in two steps: per-block
// partial sums over kRmsRows rows, then a per-column sum over the blocks in
// a fixed order (deterministic).
// ---------------------------------------------------------------------------
namespace sla2h {
namespace {

constexpr int kRmsRows = 16;  // rows per workgroup (4 per wave) in the backward's partial dw

template <int DT>
__device__ inline float ld1(const void* p, int64_t i) {
  if (DT == kF32) return static_cast<const float*>(p)[i];
  if (DT == SLA2H_DTYPE_BF16) return BF16::to_f32(static_cast<const uint16_t*>(p)[i]);
  return F16::to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <int DT>
__device__ inline void st1(void* p, int64_t i, float v) {
  if (DT == kF32)
    static_cast<float*>(p)[i] = v;
  else if (DT == SLA2H_DTYPE_BF16)
    static_cast<uint16_t*>(p)[i] = BF16::from_f32(v);
  else
    static_cast<uint16_t*>(p)[i] = F16::from_f32(v);
}
template <int DT>
__device__ inline float round_to(float v) {
  if (DT == kF32) return v;
  if (DT == SLA2H_DTYPE_BF16) return BF16::to_f32(BF16::from_f32(v));
  return F16::to_f32(F16::from_f32(v));
}
__device__ inline float wave_sum64(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <int DT, int MAXE>
__global__ __launch_bounds__(256) void rms_fwd_kernel(const void* __restrict__ X, int64_t rows, int D,
                                                      int64_t sx, const float* __restrict__ W,
                                                      float eps, float* __restrict__ Y) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int l = threadIdx.x & 63;
  float x[MAXE];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < MAXE; ++e) {
    const int c = l + 64 * e;
    x[e] = c < D ? ld1<DT>(X, row * sx + c) : 0.f;
    ss += x[e] * x[e];
  }
  const float r = 1.f / sqrtf(wave_sum64(ss) / (float)D + eps);
#pragma unroll
  for (int e = 0; e < MAXE; ++e) {
    const int c = l + 64 * e;
    if (c < D) Y[row * D + c] = round_to<DT>(x[e] * r) * W[c];
  }
}

template <int DT, int MAXE>
__global__ __launch_bounds__(256) void rms_bwd_kernel(const void* __restrict__ X, int64_t rows, int D,
                                                      int64_t sx, const float* __restrict__ W,
                                                      const float* __restrict__ DY, float eps,
                                                      void* __restrict__ DX,
                                                      float* __restrict__ DWP) {
  __shared__ float part[4][1024];
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  float dwacc[MAXE];
#pragma unroll
  for (int e = 0; e < MAXE; ++e) dwacc[e] = 0.f;
  // this wave's rows: all loads first (the rows are independent), then the math
  constexpr int R = kRmsRows / 4;
  float x[R][MAXE], dy[R][MAXE];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int64_t row = (int64_t)blockIdx.x * kRmsRows + 4 * k + w;
#pragma unroll
    for (int e = 0; e < MAXE; ++e) {
      const int c = l + 64 * e;
      const bool ok = row < rows && c < D;
      x[k][e] = ok ? ld1<DT>(X, row * sx + c) : 0.f;
      dy[k][e] = ok ? DY[row * D + c] : 0.f;
    }
  }
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int64_t row = (int64_t)blockIdx.x * kRmsRows + 4 * k + w;
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < MAXE; ++e) ss += x[k][e] * x[k][e];
    const float r = 1.f / sqrtf(wave_sum64(ss) / (float)D + eps);
    float g[MAXE];
    float gx = 0.f;
#pragma unroll
    for (int e = 0; e < MAXE; ++e) {
      const int c = l + 64 * e;
      g[e] = c < D ? round_to<DT>(dy[k][e] * W[c]) : 0.f;
      gx += g[e] * x[k][e];
      dwacc[e] += round_to<DT>(x[k][e] * r) * dy[k][e];  // rows past the end add 0
    }
    const float mgx = wave_sum64(gx) / (float)D;
    const float r3 = r * r * r;
    if (row < rows) {
#pragma unroll
      for (int e = 0; e < MAXE; ++e) {
        const int c = l + 64 * e;
        if (c < D) st1<DT>(DX, row * D + c, r * g[e] - x[k][e] * r3 * mgx);
      }
    }
  }
  // partial dw of this workgroup's rows: the four waves' sums in a fixed order
#pragma unroll
  for (int e = 0; e < MAXE; ++e) {
    const int c = l + 64 * e;
    if (c < D) part[w][c] = dwacc[e];
  }
  __syncthreads();
  for (int c = threadIdx.x; c < D; c += 256)
    DWP[(int64_t)blockIdx.x * D + c] = (part[0][c] + part[1][c]) + (part[2][c] + part[3][c]);
}

// dw[c] = sum over b of partial[b][c]: one workgroup per column, thread t
// sums b = t, t + 256, ... in order, then a fixed LDS tree (deterministic)
__global__ __launch_bounds__(256) void col_sum_kernel(const float* __restrict__ P, int64_t nb, int D,
                                                      float* __restrict__ out) {
  __shared__ float red[256];
  const int c = blockIdx.x;
  float s = 0.f;
  for (int64_t b = threadIdx.x; b < nb; b += 256) s += P[b * D + c];
  red[threadIdx.x] = s;
  __syncthreads();
#pragma unroll
  for (int h = 128; h >= 1; h >>= 1) {
    if ((int)threadIdx.x < h) red[threadIdx.x] += red[threadIdx.x + h];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[c] = red[0];
}

// Vectorised variant for D = 8 LPR (LPR a power of two <= 64 lanes per row):
// lane l of a wave owns channels 8 (l % LPR) .. +7 of row slot l / LPR, so a
// wave covers 64 / LPR rows per pass with 16-byte accesses (two for fp32).
template <int DT>
__device__ inline void ld8(const void* p, int64_t i, float (&x)[8]) {
  if (DT == kF32) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
    x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
  } else {
    Vec<DT == kF32 ? SLA2H_DTYPE_BF16 : DT>::ld(p, i, x);
  }
}
template <int DT>
__device__ inline void st8(void* p, int64_t i, const float (&x)[8]) {
  if (DT == kF32) {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(x[0], x[1], x[2], x[3]);
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i + 4) = make_float4(x[4], x[5], x[6], x[7]);
  } else {
    Vec<DT == kF32 ? SLA2H_DTYPE_BF16 : DT>::st(p, i, x);
  }
}
__device__ inline void ld8f(const float* p, int64_t i, float (&x)[8]) { ld8<kF32>(p, i, x); }
template <int LPR>
__device__ inline float group_sum(float v) {  // over the LPR lanes of a row (aligned groups)
#pragma unroll
  for (int m = LPR / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// OT: the output's type (fp32, or a 16-bit type: the fp32 result rounded once)
template <int DT, int LPR, int OT = kF32>
__global__ __launch_bounds__(256) void rms_fwd_vec_kernel(const void* __restrict__ X, int64_t rows,
                                                          int64_t sx, const float* __restrict__ W,
                                                          float eps, void* __restrict__ Y) {
  constexpr int D = 8 * LPR, RPW = 64 / LPR;
  const int l = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + l / LPR;
  const int c0 = 8 * (l % LPR);
  const bool ok = row < rows;
  float x[8];
  if (ok)
    ld8<DT>(X, row * sx + c0, x);
  else
    for (int e = 0; e < 8; ++e) x[e] = 0.f;
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  const float r = 1.f / sqrtf(group_sum<LPR>(ss) / (float)D + eps);
  float w[8], y[8];
  ld8f(W, c0, w);
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = round_to<DT>(x[e] * r) * w[e];
  if (ok) st8<OT>(Y, row * D + c0, y);
}

// backward: 4 passes of 64 / LPR rows per wave, loads first; dw partials of the
// workgroup's 16 * 64 / LPR rows
// DYT = kF32: one fp32 output gradient DY0.  DYT 16-bit: the output gradient
// is DY0 + DY1 + DY2 summed in fp32 in that order (DY1, DY2 may be null: the
// gradients of the consumers of a shared 16-bit output), and DADD (fp32, may
// be null) is added to dx (the gradient the input also receives elsewhere).
template <int DT, int LPR, int DYT = kF32>
__global__ __launch_bounds__(256) void rms_bwd_vec_kernel(const void* __restrict__ X, int64_t rows,
                                                          int64_t sx, const float* __restrict__ W,
                                                          const void* __restrict__ DY0,
                                                          const void* __restrict__ DY1,
                                                          const void* __restrict__ DY2,
                                                          const float* __restrict__ DADD, float eps,
                                                          void* __restrict__ DX,
                                                          float* __restrict__ DWP) {
  constexpr int D = 8 * LPR, RPW = 64 / LPR, P = 4;
  __shared__ float part[4][D];
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int c0 = 8 * (l % LPR);
  const int64_t row0 = (int64_t)blockIdx.x * (4 * P * RPW);
  float x[P][8], dy[P][8], wv[8], dwacc[8];
  ld8f(W, c0, wv);
#pragma unroll
  for (int e = 0; e < 8; ++e) dwacc[e] = 0.f;
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const int64_t row = row0 + ((int64_t)(k * 4 + w)) * RPW + l / LPR;
    if (row < rows) {
      ld8<DT>(X, row * sx + c0, x[k]);
      if (DYT == kF32) {
        ld8f(static_cast<const float*>(DY0), row * D + c0, dy[k]);
      } else {
        ld8<DYT>(DY0, row * D + c0, dy[k]);
        float t[8];
        if (DY1 != nullptr) {
          ld8<DYT>(DY1, row * D + c0, t);
#pragma unroll
          for (int e = 0; e < 8; ++e) dy[k][e] += t[e];
        }
        if (DY2 != nullptr) {
          ld8<DYT>(DY2, row * D + c0, t);
#pragma unroll
          for (int e = 0; e < 8; ++e) dy[k][e] += t[e];
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[k][e] = dy[k][e] = 0.f;
    }
  }
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const int64_t row = row0 + ((int64_t)(k * 4 + w)) * RPW + l / LPR;
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x[k][e] * x[k][e];
    const float r = 1.f / sqrtf(group_sum<LPR>(ss) / (float)D + eps);
    float g[8], gx = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      g[e] = round_to<DT>(dy[k][e] * wv[e]);
      gx += g[e] * x[k][e];
      dwacc[e] += round_to<DT>(x[k][e] * r) * dy[k][e];  // rows past the end add 0
    }
    const float mgx = group_sum<LPR>(gx) / (float)D;
    const float r3 = r * r * r;
    float dx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) dx[e] = r * g[e] - x[k][e] * r3 * mgx;
    if (row < rows) {
      if (DYT != kF32 && DADD != nullptr) {
        float t[8];
        ld8f(DADD, row * D + c0, t);
#pragma unroll
        for (int e = 0; e < 8; ++e) dx[e] = dx[e] + t[e];
      }
      st8<DT>(DX, row * D + c0, dx);
    }
  }
  // combine the wave's row slots (lanes l, l ^ LPR, ...), fixed order
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int m = LPR; m < 64; m <<= 1) dwacc[e] += __shfl_xor(dwacc[e], m, 64);
  if (l < LPR)
#pragma unroll
    for (int e = 0; e < 8; ++e) part[w][c0 + e] = dwacc[e];
  __syncthreads();
  for (int c = threadIdx.x; c < D; c += 256)
    DWP[(int64_t)blockIdx.x * D + c] = (part[0][c] + part[1][c]) + (part[2][c] + part[3][c]);
}

// lanes per row of the vectorised kernels for this shape, or 0
template <int DT>
int rms_vec_lpr(const void* x, int D, int64_t sx) {
  if (D % 8 || D > 512 || (D & (D - 1)) || reinterpret_cast<uintptr_t>(x) % 16 ||
      sx % (DT == kF32 ? 4 : 8))
    return 0;
  return D / 8;
}

template <int DT>
void launch_rms_fwd(const void* x, int64_t rows, int D, int64_t sx, const float* w, float eps,
                    float* y, hipStream_t st) {
  const int lpr = rms_vec_lpr<DT>(x, D, sx);
  if (lpr) {
    const unsigned g = (unsigned)((rows + 4 * (64 / lpr) - 1) / (4 * (64 / lpr)));
#define SLA2H_RMSF(LPR) rms_fwd_vec_kernel<DT, LPR><<<g, 256, 0, st>>>(x, rows, sx, w, eps, y)
    switch (lpr) {
      case 1: SLA2H_RMSF(1); return;
      case 2: SLA2H_RMSF(2); return;
      case 4: SLA2H_RMSF(4); return;
      case 8: SLA2H_RMSF(8); return;
      case 16: SLA2H_RMSF(16); return;
      case 32: SLA2H_RMSF(32); return;
      default: SLA2H_RMSF(64); return;
    }
#undef SLA2H_RMSF
  }
  const unsigned grid = (unsigned)((rows + 3) / 4);
  if (D <= 64)
    rms_fwd_kernel<DT, 1><<<grid, 256, 0, st>>>(x, rows, D, sx, w, eps, y);
  else if (D <= 256)
    rms_fwd_kernel<DT, 4><<<grid, 256, 0, st>>>(x, rows, D, sx, w, eps, y);
  else if (D <= 512)
    rms_fwd_kernel<DT, 8><<<grid, 256, 0, st>>>(x, rows, D, sx, w, eps, y);
  else
    rms_fwd_kernel<DT, 16><<<grid, 256, 0, st>>>(x, rows, D, sx, w, eps, y);
}
// rows per workgroup of the backward for this shape (partial dw rows)
template <int DT>
int64_t rms_bwd_rows_per_block(const void* x, int D, int64_t sx) {
  const int lpr = rms_vec_lpr<DT>(x, D, sx);
  return lpr ? 16 * (64 / lpr) : kRmsRows;
}

template <int DT>
void launch_rms_bwd(const void* x, int64_t rows, int D, int64_t sx, const float* w, const float* dy,
                    float eps, void* dx, float* dwp, hipStream_t st) {
  const int lpr = rms_vec_lpr<DT>(x, D, sx);
  if (lpr) {
    const int64_t rpb = 16 * (64 / lpr);
    const unsigned g = (unsigned)((rows + rpb - 1) / rpb);
#define SLA2H_RMSB(LPR) rms_bwd_vec_kernel<DT, LPR><<<g, 256, 0, st>>>(x, rows, sx, w, dy, nullptr, nullptr, nullptr, eps, dx, dwp)
    switch (lpr) {
      case 1: SLA2H_RMSB(1); return;
      case 2: SLA2H_RMSB(2); return;
      case 4: SLA2H_RMSB(4); return;
      case 8: SLA2H_RMSB(8); return;
      case 16: SLA2H_RMSB(16); return;
      case 32: SLA2H_RMSB(32); return;
      default: SLA2H_RMSB(64); return;
    }
#undef SLA2H_RMSB
  }
  const unsigned grid = (unsigned)((rows + kRmsRows - 1) / kRmsRows);
  if (D <= 64)
    rms_bwd_kernel<DT, 1><<<grid, 256, 0, st>>>(x, rows, D, sx, w, dy, eps, dx, dwp);
  else if (D <= 256)
    rms_bwd_kernel<DT, 4><<<grid, 256, 0, st>>>(x, rows, D, sx, w, dy, eps, dx, dwp);
  else if (D <= 512)
    rms_bwd_kernel<DT, 8><<<grid, 256, 0, st>>>(x, rows, D, sx, w, dy, eps, dx, dwp);
  else
    rms_bwd_kernel<DT, 16><<<grid, 256, 0, st>>>(x, rows, D, sx, w, dy, eps, dx, dwp);
}

// fp32 x, D = 8 LPR: the 16-bit-output forward and the multi-gradient backward
template <int OT>
void launch_rms_fwd16(const float* x, int64_t rows, int lpr, int64_t sx, const float* w, float eps,
                      void* y, hipStream_t st) {
  const unsigned g = (unsigned)((rows + 4 * (64 / lpr) - 1) / (4 * (64 / lpr)));
#define SLA2H_RMSF16(LPR) rms_fwd_vec_kernel<kF32, LPR, OT><<<g, 256, 0, st>>>(x, rows, sx, w, eps, y)
  switch (lpr) {
    case 1: SLA2H_RMSF16(1); return;
    case 2: SLA2H_RMSF16(2); return;
    case 4: SLA2H_RMSF16(4); return;
    case 8: SLA2H_RMSF16(8); return;
    case 16: SLA2H_RMSF16(16); return;
    case 32: SLA2H_RMSF16(32); return;
    default: SLA2H_RMSF16(64); return;
  }
#undef SLA2H_RMSF16
}
template <int DYT>
void launch_rms_bwd_sum(const float* x, int64_t rows, int lpr, int64_t sx, const float* w,
                        const void* dy0, const void* dy1, const void* dy2, const float* dadd,
                        float eps, float* dx, float* dwp, hipStream_t st) {
  const int64_t rpb = 16 * (64 / lpr);
  const unsigned g = (unsigned)((rows + rpb - 1) / rpb);
#define SLA2H_RMSBS(LPR) rms_bwd_vec_kernel<kF32, LPR, DYT><<<g, 256, 0, st>>>(x, rows, sx, w, dy0, dy1, dy2, dadd, eps, dx, dwp)
  switch (lpr) {
    case 1: SLA2H_RMSBS(1); return;
    case 2: SLA2H_RMSBS(2); return;
    case 4: SLA2H_RMSBS(4); return;
    case 8: SLA2H_RMSBS(8); return;
    case 16: SLA2H_RMSBS(16); return;
    case 32: SLA2H_RMSBS(32); return;
    default: SLA2H_RMSBS(64); return;
  }
#undef SLA2H_RMSBS
}

}  // namespace
}  // namespace sla2h

extern "C" size_t sla2h_rmsnorm_bwd_workspace_bytes(int64_t rows, int D) {
  if (rows <= 0 || D <= 0) return 0;
  return (size_t)((rows + sla2h::kRmsRows - 1) / sla2h::kRmsRows) * D * sizeof(float);
}

extern "C" int sla2h_rmsnorm_fwd(const void* x, int dtype, int64_t rows, int D, int64_t sx,
                                 const float* w, float eps, float* y, void* stream) {
  SLA2H_CHECK_ARG(x && w && y);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16 || dtype == kF32);
  SLA2H_CHECK_ARG(rows > 0 && D > 0 && D <= 1024 && sx >= D);
  SLA2H_CHECK_ARG((rows + 3) / 4 < (1ll << 31));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SLA2H_DTYPE_BF16)
    launch_rms_fwd<SLA2H_DTYPE_BF16>(x, rows, D, sx, w, eps, y, st);
  else if (dtype == SLA2H_DTYPE_F16)
    launch_rms_fwd<SLA2H_DTYPE_F16>(x, rows, D, sx, w, eps, y, st);
  else
    launch_rms_fwd<kF32>(x, rows, D, sx, w, eps, y, st);
  return (int)hipGetLastError();
}

extern "C" int sla2h_rmsnorm_bwd(const void* x, int dtype, int64_t rows, int D, int64_t sx,
                                 const float* w, const float* dy, float eps, void* dx, float* dw,
                                 void* workspace, void* stream) {
  SLA2H_CHECK_ARG(x && w && dy && dx && dw && workspace);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16 || dtype == kF32);
  SLA2H_CHECK_ARG(rows > 0 && D > 0 && D <= 1024 && sx >= D);
  const int64_t rpb = dtype == SLA2H_DTYPE_BF16 ? rms_bwd_rows_per_block<SLA2H_DTYPE_BF16>(x, D, sx)
                      : dtype == SLA2H_DTYPE_F16 ? rms_bwd_rows_per_block<SLA2H_DTYPE_F16>(x, D, sx)
                                                 : rms_bwd_rows_per_block<kF32>(x, D, sx);
  const int64_t nb = (rows + rpb - 1) / rpb;
  SLA2H_CHECK_ARG(nb < (1ll << 31));
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* dwp = static_cast<float*>(workspace);
  if (dtype == SLA2H_DTYPE_BF16)
    launch_rms_bwd<SLA2H_DTYPE_BF16>(x, rows, D, sx, w, dy, eps, dx, dwp, st);
  else if (dtype == SLA2H_DTYPE_F16)
    launch_rms_bwd<SLA2H_DTYPE_F16>(x, rows, D, sx, w, dy, eps, dx, dwp, st);
  else
    launch_rms_bwd<kF32>(x, rows, D, sx, w, dy, eps, dx, dwp, st);
  int err = (int)hipGetLastError();
  if (err) return err;
  col_sum_kernel<<<D, 256, 0, st>>>(dwp, nb, D, dw);
  return (int)hipGetLastError();
}

extern "C" int sla2h_rmsnorm_fwd16(const float* x, int64_t rows, int D, int64_t sx,
                                   const float* w, float eps, int out_dtype, void* y,
                                   void* stream) {
  SLA2H_CHECK_ARG(x && w && y);
  SLA2H_CHECK_ARG(out_dtype == SLA2H_DTYPE_F16 || out_dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(rows > 0 && D > 0 && sx >= D);
  const int lpr = rms_vec_lpr<kF32>(x, D, sx);
  SLA2H_CHECK_ARG(lpr > 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0);
  SLA2H_CHECK_ARG((rows + 4 * (64 / lpr) - 1) / (4 * (64 / lpr)) < (1ll << 31));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (out_dtype == SLA2H_DTYPE_BF16)
    launch_rms_fwd16<SLA2H_DTYPE_BF16>(x, rows, lpr, sx, w, eps, y, st);
  else
    launch_rms_fwd16<SLA2H_DTYPE_F16>(x, rows, lpr, sx, w, eps, y, st);
  return (int)hipGetLastError();
}

extern "C" int sla2h_rmsnorm_bwd_sum(const float* x, int64_t rows, int D, int64_t sx,
                                     const float* w, const void* dy0, const void* dy1,
                                     const void* dy2, int dy_dtype, const float* dadd, float eps,
                                     float* dx, float* dw, void* workspace, void* stream) {
  SLA2H_CHECK_ARG(x && w && dy0 && dx && dw && workspace);
  SLA2H_CHECK_ARG(dy_dtype == SLA2H_DTYPE_F16 || dy_dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(rows > 0 && D > 0 && sx >= D);
  const int lpr = rms_vec_lpr<kF32>(x, D, sx);
  SLA2H_CHECK_ARG(lpr > 0);
  for (const void* p : {dy0, dy1, dy2, static_cast<const void*>(dadd), static_cast<const void*>(dx)})
    SLA2H_CHECK_ARG(reinterpret_cast<uintptr_t>(p) % 16 == 0);
  const int64_t rpb = 16 * (64 / lpr);
  const int64_t nb = (rows + rpb - 1) / rpb;
  SLA2H_CHECK_ARG(nb < (1ll << 31));
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* dwp = static_cast<float*>(workspace);
  if (dy_dtype == SLA2H_DTYPE_BF16)
    launch_rms_bwd_sum<SLA2H_DTYPE_BF16>(x, rows, lpr, sx, w, dy0, dy1, dy2, dadd, eps, dx, dwp, st);
  else
    launch_rms_bwd_sum<SLA2H_DTYPE_F16>(x, rows, lpr, sx, w, dy0, dy1, dy2, dadd, eps, dx, dwp, st);
  int err = (int)hipGetLastError();
  if (err) return err;
  col_sum_kernel<<<D, 256, 0, st>>>(dwp, nb, D, dw);
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// RoPE of the training forward (models/imf_dit_video.py:266-284): channel pairs
// (2i, 2i+1) of x (b, l, H, hd) rotated by the angle of token l, in fp32, cast
// back: (re c - im s, re s + im c).  The backward is the rotation by -angle of
// the output gradient (inverse = 1): (dre c + dim s, -dre s + dim c).  x may be
// a strided view (unit channel stride); out is contiguous (b, l, H, hd).
// One thread per channel pair.
// ---------------------------------------------------------------------------
namespace sla2h {
namespace {

template <int DT>
__global__ __launch_bounds__(256) void rope_kernel(const void* __restrict__ X, int64_t B, int64_t L,
                                                   int H, int hd, int64_t sb, int64_t sl,
                                                   int64_t sh, const float* __restrict__ COS,
                                                   const float* __restrict__ SIN, float sgn,
                                                   void* __restrict__ OUT) {
  const int hp = hd >> 1;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= B * L * H * hp) return;
  const int i = (int)(idx % hp);
  int64_t t = idx / hp;
  const int h = (int)(t % H);
  t /= H;
  const int64_t l = t % L, b = t / L;
  const int64_t xi = b * sb + l * sl + h * sh + 2 * i;
  const float re = ld1<DT>(X, xi), im = ld1<DT>(X, xi + 1);
  const float c = COS[l * hp + i], s = sgn * SIN[l * hp + i];
  const int64_t oi = 2 * idx;
  st1<DT>(OUT, oi, re * c - im * s);
  st1<DT>(OUT, oi + 1, re * s + im * c);
}

}  // namespace
}  // namespace sla2h

extern "C" int sla2h_rope(const void* x, int dtype, int64_t B, int64_t L, int H, int hd,
                          int64_t sb, int64_t sl, int64_t sh, const float* cos_t,
                          const float* sin_t, int inverse, void* out, void* stream) {
  SLA2H_CHECK_ARG(x && cos_t && sin_t && out);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16 || dtype == kF32);
  SLA2H_CHECK_ARG(B > 0 && L > 0 && H > 0 && hd > 0 && hd % 2 == 0);
  const int64_t n = B * L * H * (hd / 2);
  const unsigned grid = grid_of(n);
  SLA2H_CHECK_ARG(grid > 0);
  const float sgn = inverse ? -1.f : 1.f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SLA2H_DTYPE_BF16)
    rope_kernel<SLA2H_DTYPE_BF16><<<grid, 256, 0, st>>>(x, B, L, H, hd, sb, sl, sh, cos_t, sin_t, sgn, out);
  else if (dtype == SLA2H_DTYPE_F16)
    rope_kernel<SLA2H_DTYPE_F16><<<grid, 256, 0, st>>>(x, B, L, H, hd, sb, sl, sh, cos_t, sin_t, sgn, out);
  else
    rope_kernel<kF32><<<grid, 256, 0, st>>>(x, B, L, H, hd, sb, sl, sh, cos_t, sin_t, sgn, out);
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// ReZero residual of the block (models/imf_dit_video.py:529-532):
// y = x + a s with x fp32 (rows, D), a (rows, D) 16-bit or fp32, s fp32 (D);
// the product and the sum round separately (no contraction), as in the eager
// expression.  Backward: da = round_a(dy s), ds = sum over rows of dy a (per
// 16-row-block partials, then the fixed-order column sum), dx = dy (no kernel).
// ---------------------------------------------------------------------------
namespace sla2h {
namespace {

template <int DT>
__global__ __launch_bounds__(256) void residual_fwd_kernel(const float* __restrict__ X,
                                                           const void* __restrict__ A,
                                                           const float* __restrict__ S,
                                                           int64_t rows, int D,
                                                           float* __restrict__ Y) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * D) return;
  const int c = (int)(idx % D);
  const float p = ld1<DT>(A, idx) * S[c];
  Y[idx] = X[idx] + p;
}

// eight consecutive elements per thread (D % 8 == 0, 16-byte aligned rows):
// the same arithmetic with 16-byte accesses
template <int DT>
__global__ __launch_bounds__(256) void residual_fwd8_kernel(const float* __restrict__ X,
                                                            const void* __restrict__ A,
                                                            const float* __restrict__ S,
                                                            int64_t n8, int D,
                                                            float* __restrict__ Y) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const int c = (int)((8 * i) % D);
  float x[8], a[8], sc[8], y[8];
  ld8<kF32>(X, 8 * i, x);
  ld8<DT>(A, 8 * i, a);
  ld8<kF32>(S, c, sc);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = a[e] * sc[e];
    y[e] = x[e] + p;
  }
  st8<kF32>(Y, 8 * i, y);
}

// one workgroup per 16 rows, thread t owns columns t, t + 256, ...
template <int DT>
__global__ __launch_bounds__(256) void residual_bwd_kernel(const float* __restrict__ DY,
                                                           const void* __restrict__ A,
                                                           const float* __restrict__ S,
                                                           int64_t rows, int D,
                                                           void* __restrict__ DA,
                                                           float* __restrict__ DSP) {
#pragma clang fp contract(off)
  const int64_t r0 = (int64_t)blockIdx.x * kRmsRows;
  for (int c = threadIdx.x; c < D; c += 256) {
    const float s = S[c];
    float acc = 0.f;
    for (int k = 0; k < kRmsRows; ++k) {
      const int64_t row = r0 + k;
      if (row >= rows) break;
      const int64_t i = row * D + c;
      const float dy = DY[i];
      st1<DT>(DA, i, dy * s);
      acc += dy * ld1<DT>(A, i);
    }
    DSP[(int64_t)blockIdx.x * D + c] = acc;
  }
}

}  // namespace
}  // namespace sla2h

extern "C" int sla2h_residual_scale_fwd(const float* x, const void* a, int dtype, const float* s,
                                        int64_t rows, int D, float* y, void* stream) {
  SLA2H_CHECK_ARG(x && a && s && y && rows > 0 && D > 0);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16 || dtype == kF32);
  const unsigned grid = grid_of(rows * D);
  SLA2H_CHECK_ARG(grid > 0);
  hipStream_t st = static_cast<hipStream_t>(stream);
  bool wide = D % 8 == 0;
  for (const void* p : {static_cast<const void*>(x), a, static_cast<const void*>(s),
                        static_cast<const void*>(y)})
    wide = wide && reinterpret_cast<uintptr_t>(p) % 16 == 0;
  if (wide) {
    const unsigned g8 = grid_of(rows * D / 8);
    if (dtype == SLA2H_DTYPE_BF16)
      residual_fwd8_kernel<SLA2H_DTYPE_BF16><<<g8, 256, 0, st>>>(x, a, s, rows * D / 8, D, y);
    else if (dtype == SLA2H_DTYPE_F16)
      residual_fwd8_kernel<SLA2H_DTYPE_F16><<<g8, 256, 0, st>>>(x, a, s, rows * D / 8, D, y);
    else
      residual_fwd8_kernel<kF32><<<g8, 256, 0, st>>>(x, a, s, rows * D / 8, D, y);
    return (int)hipGetLastError();
  }
  if (dtype == SLA2H_DTYPE_BF16)
    residual_fwd_kernel<SLA2H_DTYPE_BF16><<<grid, 256, 0, st>>>(x, a, s, rows, D, y);
  else if (dtype == SLA2H_DTYPE_F16)
    residual_fwd_kernel<SLA2H_DTYPE_F16><<<grid, 256, 0, st>>>(x, a, s, rows, D, y);
  else
    residual_fwd_kernel<kF32><<<grid, 256, 0, st>>>(x, a, s, rows, D, y);
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Output gate of the MLA sublayer (models/imf_dit_video.py:466, attn *
// sigmoid(g) on 16-bit tensors under autocast), eight elements per thread:
//   s = round16(1 / (1 + exp(-g))), out = round16(a s);
//   backward: da = round16(dout s), ds = round16(dout a),
//   dg = round16(round16(ds round16(1 - s)) s)  (s recomputed from g,
//   bit-identical; torch's GPU sigmoid backward computes a (1 - b) b in the
//   16-bit type itself, one rounding per operation).
// ---------------------------------------------------------------------------
namespace sla2h {
namespace {

template <int DT>
__device__ inline float gate_sig(float g) {
  return round_to<DT>(1.f / (1.f + expf(-g)));
}

template <int DT>
__global__ __launch_bounds__(256) void gate_fwd_kernel(const void* __restrict__ A,
                                                       const void* __restrict__ G, int64_t n8,
                                                       void* __restrict__ O) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  float a[8], g[8], o[8];
  Vec<DT>::ld(A, 8 * i, a);
  Vec<DT>::ld(G, 8 * i, g);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = a[e] * gate_sig<DT>(g[e]);
  Vec<DT>::st(O, 8 * i, o);
}

template <int DT>
__global__ __launch_bounds__(256) void gate_bwd_kernel(const void* __restrict__ DO,
                                                       const void* __restrict__ A,
                                                       const void* __restrict__ G, int64_t n8,
                                                       void* __restrict__ DA,
                                                       void* __restrict__ DG) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  float d[8], a[8], g[8], da[8], dg[8];
  Vec<DT>::ld(DO, 8 * i, d);
  Vec<DT>::ld(A, 8 * i, a);
  Vec<DT>::ld(G, 8 * i, g);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float sg = gate_sig<DT>(g[e]);
    da[e] = d[e] * sg;
    const float ds = round_to<DT>(d[e] * a[e]);
    dg[e] = round_to<DT>(ds * round_to<DT>(1.f - sg)) * sg;
  }
  Vec<DT>::st(DA, 8 * i, da);
  Vec<DT>::st(DG, 8 * i, dg);
}

}  // namespace
}  // namespace sla2h

extern "C" int sla2h_gate_mul_fwd(const void* a, const void* g, int dtype, int64_t n, void* out,
                                  void* stream) {
  SLA2H_CHECK_ARG(a && g && out && n > 0 && n % 8 == 0);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  for (const void* p : {a, g, static_cast<const void*>(out)})
    SLA2H_CHECK_ARG(reinterpret_cast<uintptr_t>(p) % 16 == 0);
  const unsigned grid = grid_of(n / 8);
  SLA2H_CHECK_ARG(grid > 0);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SLA2H_DTYPE_BF16)
    gate_fwd_kernel<SLA2H_DTYPE_BF16><<<grid, 256, 0, st>>>(a, g, n / 8, out);
  else
    gate_fwd_kernel<SLA2H_DTYPE_F16><<<grid, 256, 0, st>>>(a, g, n / 8, out);
  return (int)hipGetLastError();
}

extern "C" int sla2h_gate_mul_bwd(const void* dout, const void* a, const void* g, int dtype,
                                  int64_t n, void* da, void* dg, void* stream) {
  SLA2H_CHECK_ARG(dout && a && g && da && dg && n > 0 && n % 8 == 0);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  for (const void* p : {dout, a, g, static_cast<const void*>(da), static_cast<const void*>(dg)})
    SLA2H_CHECK_ARG(reinterpret_cast<uintptr_t>(p) % 16 == 0);
  const unsigned grid = grid_of(n / 8);
  SLA2H_CHECK_ARG(grid > 0);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SLA2H_DTYPE_BF16)
    gate_bwd_kernel<SLA2H_DTYPE_BF16><<<grid, 256, 0, st>>>(dout, a, g, n / 8, da, dg);
  else
    gate_bwd_kernel<SLA2H_DTYPE_F16><<<grid, 256, 0, st>>>(dout, a, g, n / 8, da, dg);
  return (int)hipGetLastError();
}

extern "C" size_t sla2h_residual_scale_bwd_workspace_bytes(int64_t rows, int D) {
  return sla2h_rmsnorm_bwd_workspace_bytes(rows, D);
}

extern "C" int sla2h_residual_scale_bwd(const float* dy, const void* a, int dtype, const float* s,
                                        int64_t rows, int D, void* da, float* ds, void* workspace,
                                        void* stream) {
  SLA2H_CHECK_ARG(dy && a && s && da && ds && workspace && rows > 0 && D > 0);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16 || dtype == kF32);
  const int64_t nb = (rows + kRmsRows - 1) / kRmsRows;
  SLA2H_CHECK_ARG(nb < (1ll << 31));
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* dsp = static_cast<float*>(workspace);
  if (dtype == SLA2H_DTYPE_BF16)
    residual_bwd_kernel<SLA2H_DTYPE_BF16><<<(unsigned)nb, 256, 0, st>>>(dy, a, s, rows, D, da, dsp);
  else if (dtype == SLA2H_DTYPE_F16)
    residual_bwd_kernel<SLA2H_DTYPE_F16><<<(unsigned)nb, 256, 0, st>>>(dy, a, s, rows, D, da, dsp);
  else
    residual_bwd_kernel<kF32><<<(unsigned)nb, 256, 0, st>>>(dy, a, s, rows, D, da, dsp);
  int err = (int)hipGetLastError();
  if (err) return err;
  col_sum_kernel<<<D, 256, 0, st>>>(dsp, nb, D, ds);
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Attention operands and output gate of the MLA sublayer around a tile-major
// SLA2 op (models/imf_dit_video.py:458-466 with models/sla2_cube_qat.py:
// 340-350, 397-400).  The sublayer builds q = cat([q_nope, q_rope]) and
// k = cat([k_nope, k_rope shared by the heads]), each (B, L, H, 64), where the
// nope halves are the per-head RMSNorm outputs (fp32: the norm's 16-bit
// result times its fp32 weight) and the rope halves and v are 16-bit; the op
// takes permute(0, 2, 1, 3).half() of q, k, v and returns (B, H, L, 64) fp16
// rows, which go back through permute(...).to(fp32) and the gate
// attn * sigmoid(g) into the output projection's autocast cast.
//
// attn_in: the three operand tensors straight from their halves into the
// op's fp16 rows, eight channels per thread (channels 0..31 from the "lo"
// half, 32..63 from the "hi" half; a half is addressed by (b, t, h) strides
// in elements, h stride 0 for the band the heads share).  Every value is
// converted once to fp16, as .half() of the exact concatenation does.  The
// backward writes each half's gradient in the half's own dtype: fp32 exactly,
// a 16-bit half rounded once from fp16 (the concatenation's fp32 gradient cast
// back to the half's dtype); the shared band's gradient is the fp32 sum over
// the heads, in head order, of the per-head 16-bit gradients, rounded once
// (the expand's backward sum).
//
// attn_gate: out = round16(fp32(o) s), s = round16(sigmoid(g)) (the gate's
// fp32 product, then the output projection's cast to the autocast dtype);
// backward from the projection's 16-bit input gradient d:
//   do = fp16(d s)  (the gate's fp32 da, cast back to the op's fp16 output),
//   dg = round16(round16(ds round16(1 - s)) s),  ds = round16(d fp32(o))
// (the sigmoid output is 16-bit, so its gradient is rounded to 16 bits and
// torch's sigmoid backward runs in the 16-bit type).
// ---------------------------------------------------------------------------
namespace sla2h {
namespace {

struct HalfRef {  // one 32-channel half of an operand, (b, t, h) strides in elements
  const void* p;
  int64_t sb, st, sh;
};
struct HalfOut {
  void* p;
  int64_t sb, st, sh;
};

// thread i: output row (b, h, t) = i >> 3 of the (B, H, L, 64) fp16 operand,
// channels 8 (i & 7) ..
template <int LO, int HI>
__global__ __launch_bounds__(256) void attn_in_fwd_kernel(HalfRef lo, HalfRef hi, int H, int L,
                                                          int n8, uint16_t* __restrict__ out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const int c8 = i & 7, row = i >> 3;
  const int t = row % L, bh = row / L;
  const int h = bh % H, b = bh / H;
  float x[8];
  if (c8 < 4)
    ld8<LO>(lo.p, b * lo.sb + t * lo.st + h * lo.sh + 8 * c8, x);
  else
    ld8<HI>(hi.p, b * hi.sb + t * hi.st + h * hi.sh + 8 * (c8 - 4), x);
  st8<SLA2H_DTYPE_F16>(out, 8 * (int64_t)i, x);
}

// thread i: token (b, t), head h, channels 8 c8 .. in (c8, h, t, b) order, so
// the halves' (B, L, H, 32) gradients are written contiguously.  SUMHI: the
// hi half is shared by the heads; the h = 0 thread of each (b, t, c8) sums it.
template <int LO, int HI, bool SUMHI>
__global__ __launch_bounds__(256) void attn_in_bwd_kernel(const uint16_t* __restrict__ dout,
                                                          HalfOut lo, HalfOut hi, int H, int L,
                                                          int n8) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const int c8 = i & 7, rest = i >> 3;
  const int h = rest % H, tok = rest / H;
  const int t = tok % L, b = tok / L;
  float x[8];
  if (c8 < 4) {
    ld8<SLA2H_DTYPE_F16>(dout, ((int64_t)(b * H + h) * L + t) * 64 + 8 * c8, x);
    st8<LO>(lo.p, b * lo.sb + t * lo.st + h * lo.sh + 8 * c8, x);
  } else if (!SUMHI) {
    ld8<SLA2H_DTYPE_F16>(dout, ((int64_t)(b * H + h) * L + t) * 64 + 8 * c8, x);
    st8<HI>(hi.p, b * hi.sb + t * hi.st + h * hi.sh + 8 * (c8 - 4), x);
  } else if (h == 0) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int hh = 0; hh < H; ++hh) {
      ld8<SLA2H_DTYPE_F16>(dout, ((int64_t)(b * H + hh) * L + t) * 64 + 8 * c8, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += round_to<HI>(x[e]);
    }
    st8<HI>(hi.p, b * hi.sb + t * hi.st + 8 * (c8 - 4), acc);
  }
}

// thread i: token (b, t), head h, channels 8 c8 .. (c8, h, t, b) order, i.e.
// element 8 i of the (B, L, H * 64) gate and output
template <int DT>
__global__ __launch_bounds__(256) void attn_gate_fwd_kernel(const uint16_t* __restrict__ o,
                                                            const void* __restrict__ g, int H,
                                                            int L, int n8, void* __restrict__ out) {
#pragma clang fp contract(off)
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const int c8 = i & 7, rest = i >> 3;
  const int h = rest % H, tok = rest / H;
  const int t = tok % L, b = tok / L;
  float a[8], gv[8], y[8];
  ld8<SLA2H_DTYPE_F16>(o, ((int64_t)(b * H + h) * L + t) * 64 + 8 * c8, a);
  ld8<DT>(g, 8 * (int64_t)i, gv);
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = a[e] * gate_sig<DT>(gv[e]);
  st8<DT>(out, 8 * (int64_t)i, y);
}

template <int DT>
__global__ __launch_bounds__(256) void attn_gate_bwd_kernel(const void* __restrict__ dy,
                                                            const uint16_t* __restrict__ o,
                                                            const void* __restrict__ g, int H,
                                                            int L, int n8,
                                                            uint16_t* __restrict__ dout,
                                                            void* __restrict__ dg) {
#pragma clang fp contract(off)
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const int c8 = i & 7, rest = i >> 3;
  const int h = rest % H, tok = rest / H;
  const int t = tok % L, b = tok / L;
  const int64_t oi = ((int64_t)(b * H + h) * L + t) * 64 + 8 * c8;
  float d[8], a[8], gv[8], da[8], dgv[8];
  ld8<DT>(dy, 8 * (int64_t)i, d);
  ld8<SLA2H_DTYPE_F16>(o, oi, a);
  ld8<DT>(g, 8 * (int64_t)i, gv);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float sg = gate_sig<DT>(gv[e]);
    da[e] = d[e] * sg;
    const float ds = round_to<DT>(d[e] * a[e]);
    dgv[e] = round_to<DT>(ds * round_to<DT>(1.f - sg)) * sg;
  }
  st8<SLA2H_DTYPE_F16>(dout, oi, da);
  st8<DT>(dg, 8 * (int64_t)i, dgv);
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }
bool half_ok(const void* p, int dt, int64_t sb, int64_t st, int64_t sh) {
  // 16-byte accesses: the base and every stride a multiple of 16 bytes
  const int64_t es = dt == kF32 ? 4 : 2;
  return p != nullptr && aligned16(p) && (sb * es) % 16 == 0 && (st * es) % 16 == 0 &&
         (sh * es) % 16 == 0 && sb >= 0 && st >= 0 && sh >= 0;
}
bool dt_ok(int dt, bool allow_f32) {
  return dt == SLA2H_DTYPE_F16 || dt == SLA2H_DTYPE_BF16 || (allow_f32 && dt == kF32);
}

// dispatch over (lo dtype in {f16, bf16, f32}) x (hi dtype in {f16, bf16})
template <typename F>
void attn_in_dispatch(int lo_dt, int hi_dt, F&& f) {
  auto hi = [&](auto lo_c) {
    if (hi_dt == SLA2H_DTYPE_BF16)
      f(lo_c, std::integral_constant<int, SLA2H_DTYPE_BF16>{});
    else
      f(lo_c, std::integral_constant<int, SLA2H_DTYPE_F16>{});
  };
  if (lo_dt == kF32)
    hi(std::integral_constant<int, kF32>{});
  else if (lo_dt == SLA2H_DTYPE_BF16)
    hi(std::integral_constant<int, SLA2H_DTYPE_BF16>{});
  else
    hi(std::integral_constant<int, SLA2H_DTYPE_F16>{});
}

}  // namespace
}  // namespace sla2h

extern "C" int sla2h_attn_in_fwd(const void* lo, int lo_dtype, int64_t lo_sb, int64_t lo_st,
                                 int64_t lo_sh, const void* hi, int hi_dtype, int64_t hi_sb,
                                 int64_t hi_st, int64_t hi_sh, int B, int H, int64_t L, void* out,
                                 void* stream) {
  SLA2H_CHECK_ARG(dt_ok(lo_dtype, true) && dt_ok(hi_dtype, false));
  SLA2H_CHECK_ARG(half_ok(lo, lo_dtype, lo_sb, lo_st, lo_sh));
  SLA2H_CHECK_ARG(half_ok(hi, hi_dtype, hi_sb, hi_st, hi_sh));
  SLA2H_CHECK_ARG(out && aligned16(out) && B > 0 && H > 0 && L > 0);
  const int64_t n8 = (int64_t)B * H * L * 8;
  SLA2H_CHECK_ARG(n8 < (1ll << 31));
  const unsigned grid = grid_of(n8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const HalfRef rl{lo, lo_sb, lo_st, lo_sh}, rh{hi, hi_sb, hi_st, hi_sh};
  attn_in_dispatch(lo_dtype, hi_dtype, [&](auto lc, auto hc) {
    attn_in_fwd_kernel<decltype(lc)::value, decltype(hc)::value><<<grid, 256, 0, s>>>(
        rl, rh, H, (int)L, (int)n8, static_cast<uint16_t*>(out));
  });
  return (int)hipGetLastError();
}

extern "C" int sla2h_attn_in_bwd(const void* dout, void* dlo, int lo_dtype, int64_t lo_sb,
                                 int64_t lo_st, int64_t lo_sh, void* dhi, int hi_dtype,
                                 int64_t hi_sb, int64_t hi_st, int64_t hi_sh, int B, int H,
                                 int64_t L, void* stream) {
  SLA2H_CHECK_ARG(dt_ok(lo_dtype, true) && dt_ok(hi_dtype, false));
  SLA2H_CHECK_ARG(dout && aligned16(dout) && B > 0 && H > 0 && L > 0);
  SLA2H_CHECK_ARG(half_ok(dlo, lo_dtype, lo_sb, lo_st, lo_sh));
  SLA2H_CHECK_ARG(half_ok(dhi, hi_dtype, hi_sb, hi_st, hi_sh));
  const int64_t n8 = (int64_t)B * H * L * 8;
  SLA2H_CHECK_ARG(n8 < (1ll << 31));
  const unsigned grid = grid_of(n8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const HalfOut rl{dlo, lo_sb, lo_st, lo_sh}, rh{dhi, hi_sb, hi_st, hi_sh};
  auto d = static_cast<const uint16_t*>(dout);
  attn_in_dispatch(lo_dtype, hi_dtype, [&](auto lc, auto hc) {
    constexpr int LO = decltype(lc)::value, HI = decltype(hc)::value;
    if (hi_sh == 0)
      attn_in_bwd_kernel<LO, HI, true><<<grid, 256, 0, s>>>(d, rl, rh, H, (int)L, (int)n8);
    else
      attn_in_bwd_kernel<LO, HI, false><<<grid, 256, 0, s>>>(d, rl, rh, H, (int)L, (int)n8);
  });
  return (int)hipGetLastError();
}

extern "C" int sla2h_attn_gate_fwd(const void* o, const void* g, int dtype, int B, int H,
                                   int64_t L, void* out, void* stream) {
  SLA2H_CHECK_ARG(o && g && out && aligned16(o) && aligned16(g) && aligned16(out));
  SLA2H_CHECK_ARG(dt_ok(dtype, false) && B > 0 && H > 0 && L > 0);
  const int64_t n8 = (int64_t)B * H * L * 8;
  SLA2H_CHECK_ARG(n8 < (1ll << 31));
  const unsigned grid = grid_of(n8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto op = static_cast<const uint16_t*>(o);
  if (dtype == SLA2H_DTYPE_BF16)
    attn_gate_fwd_kernel<SLA2H_DTYPE_BF16><<<grid, 256, 0, s>>>(op, g, H, (int)L, (int)n8, out);
  else
    attn_gate_fwd_kernel<SLA2H_DTYPE_F16><<<grid, 256, 0, s>>>(op, g, H, (int)L, (int)n8, out);
  return (int)hipGetLastError();
}

extern "C" int sla2h_attn_gate_bwd(const void* dy, const void* o, const void* g, int dtype, int B,
                                   int H, int64_t L, void* dout, void* dg, void* stream) {
  SLA2H_CHECK_ARG(dy && o && g && dout && dg);
  for (const void* p : {dy, o, g, static_cast<const void*>(dout), static_cast<const void*>(dg)})
    SLA2H_CHECK_ARG(aligned16(p));
  SLA2H_CHECK_ARG(dt_ok(dtype, false) && B > 0 && H > 0 && L > 0);
  const int64_t n8 = (int64_t)B * H * L * 8;
  SLA2H_CHECK_ARG(n8 < (1ll << 31));
  const unsigned grid = grid_of(n8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto op = static_cast<const uint16_t*>(o);
  auto dp = static_cast<uint16_t*>(dout);
  if (dtype == SLA2H_DTYPE_BF16)
    attn_gate_bwd_kernel<SLA2H_DTYPE_BF16><<<grid, 256, 0, s>>>(dy, op, g, H, (int)L, (int)n8, dp, dg);
  else
    attn_gate_bwd_kernel<SLA2H_DTYPE_F16><<<grid, 256, 0, s>>>(dy, op, g, H, (int)L, (int)n8, dp, dg);
  return (int)hipGetLastError();
}
