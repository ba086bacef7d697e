// Elementwise JVP stages of the MLA attention sublayer and the MLP sublayer
// around the SLA2 op (models/mla_jvp_fast.py:53-228 with the kernels of
// models/triton_mla_block_jvp.py:237-498), gfx950.  All are HBM-bound row
// kernels: one wave64 per token row, fp32 arithmetic, 16-bit (or fp32) I/O.
// Primal and tangent rows are processed together (the JVP of each stage needs
// both), the GEMMs between the stages run on hipBLASLt over the stacked
// [primal; tangent] rows.
//
//   rmsnorm_jvp   y = w x / r, dy = w (dx / r - x mean(x dx) / r^3),
//                 r = sqrt(mean(x^2) + eps)                        (:237-268)
//   qkv_prep      per head: RMSNorm JVP of the nope band, RoPE rotation of the
//                 rope band (pairs (2i, 2i+1)); the key's rope band is the
//                 shared k_rope of the token, broadcast over heads; v copied.
//                 Written straight into the attention op's (B, H, L, 64)
//                 layout, optionally at a permuted token position
//                 (tile-major order of the cube op)          (:279-425)
//   out_gate      a sigmoid(z), da sigmoid(z) + a sigmoid'(z) dz, reading the
//                 attention output back from (B, H, L, dv) at the same
//                 positions                                   (:480-498)
//   situ_jvp      h = situ(g) u, dh = situ'(g) dg u + situ(g) du,
//                 situ(g) = beta tanh(g / beta) sigmoid(g)    (:437-471)
#include "common.h"

namespace sla2h {

namespace {

template <int DT>
struct IO;
template <>
struct IO<SLA2H_DTYPE_F16> {
  __device__ static float ld(const void* p, int64_t i) {
    return F16::to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  __device__ static void st(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = F16::from_f32(v);
  }
  __device__ static float rt(float v) { return F16::to_f32(F16::from_f32(v)); }
  // elements i, i + 1 (i even, 4-byte aligned) as one 32-bit access
  __device__ static float2 ld2(const void* p, int64_t i) {
    const uint32_t u = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p) + i);
    return make_float2(F16::to_f32((uint16_t)(u & 0xffff)), F16::to_f32((uint16_t)(u >> 16)));
  }
  __device__ static void st2(void* p, int64_t i, float a, float b) {
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p) + i) =
        (uint32_t)F16::from_f32(a) | ((uint32_t)F16::from_f32(b) << 16);
  }
};
template <>
struct IO<SLA2H_DTYPE_BF16> {
  __device__ static float ld(const void* p, int64_t i) {
    return BF16::to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  __device__ static void st(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = BF16::from_f32(v);
  }
  __device__ static float rt(float v) { return BF16::to_f32(BF16::from_f32(v)); }
  // elements i, i + 1 (i even, 4-byte aligned) as one 32-bit access
  __device__ static float2 ld2(const void* p, int64_t i) {
    const uint32_t u = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p) + i);
    return make_float2(BF16::to_f32((uint16_t)(u & 0xffff)), BF16::to_f32((uint16_t)(u >> 16)));
  }
  __device__ static void st2(void* p, int64_t i, float a, float b) {
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p) + i) =
        (uint32_t)BF16::from_f32(a) | ((uint32_t)BF16::from_f32(b) << 16);
  }
};
constexpr int kF32 = 2;  // fp32 I/O code used by these kernels only
template <>
struct IO<kF32> {
  __device__ static float ld(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
  __device__ static void st(void* p, int64_t i, float v) { static_cast<float*>(p)[i] = v; }
};

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// 16-lane group sum (one head's 32-channel band is two values per lane over 16 lanes)
__device__ inline float sum16(float v) {
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

__device__ inline float sigmoidf_(float x) { return 1.f / (1.f + __expf(-x)); }

// ---------------------------------------------------------------------------
template <int TI, int TO, int MAXE>
__global__ __launch_bounds__(256) void rmsnorm_jvp_kernel(const void* __restrict__ X,
                                                         const void* __restrict__ DX,
                                                         const float* __restrict__ W,
                                                         int64_t rows, int D, int64_t sx,
                                                         void* __restrict__ Y,
                                                         void* __restrict__ DY, int64_t sy,
                                                         float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int l = threadIdx.x & 63;
  float x[MAXE], dx[MAXE];
  float ss = 0.f, sxd = 0.f;
#pragma unroll
  for (int e = 0; e < MAXE; ++e) {
    const int c = l + 64 * e;
    x[e] = dx[e] = 0.f;
    if (c < D) {
      x[e] = IO<TI>::ld(X, row * sx + c);
      dx[e] = IO<TI>::ld(DX, row * sx + c);
    }
    ss += x[e] * x[e];
    sxd += x[e] * dx[e];
  }
  ss = wave_sum(ss);
  sxd = wave_sum(sxd);
  const float inv_r = 1.f / sqrtf(ss / (float)D + eps);
  const float mxdx = sxd / (float)D;
  const float k3 = mxdx * inv_r * inv_r * inv_r;
#pragma unroll
  for (int e = 0; e < MAXE; ++e) {
    const int c = l + 64 * e;
    if (c < D) {
      const float w = W[c];
      IO<TO>::st(Y, row * sy + c, w * x[e] * inv_r);
      IO<TO>::st(DY, row * sy + c, w * (dx[e] * inv_r - x[e] * k3));
    }
  }
}

// ---------------------------------------------------------------------------
// 8 16-bit values <-> one 16-byte word (element 2j in the low half of word j)
template <int DT>
struct T16Of;
template <>
struct T16Of<SLA2H_DTYPE_F16> {
  using T = F16;
};
template <>
struct T16Of<SLA2H_DTYPE_BF16> {
  using T = BF16;
};
template <int DT>
__device__ inline void unpack8(const uint4& u, float (&x)[8]) {
  using T = typename T16Of<DT>::T;
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[2 * j] = T::to_f32((uint16_t)(w[j] & 0xffff));
    x[2 * j + 1] = T::to_f32((uint16_t)(w[j] >> 16));
  }
}
template <int DT>
__device__ inline uint4 pack8(const float (&x)[8]) {
  using T = typename T16Of<DT>::T;
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    w[j] = (uint32_t)T::from_f32(x[2 * j]) | ((uint32_t)T::from_f32(x[2 * j + 1]) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// One wave per token row (b, s), heads in groups of 8: lane l = 8 hh + c works
// on 16-byte chunk c (channels 8c..8c+7) of head 8 g + hh for every operand,
// so each load and store of the wave is one 16-byte access per lane.
// dn = dr = 32, dv = 64 (qk head dim 64): chunks 0-3 are the nope band
// (RMSNorm over the head's four nope chunks: xor 1, 2 in the lane group),
// chunks 4-7 the rope band (q's own, k's shared band from KR, rotated by
// (cos, sin)[s][4 (c - 4) + j] on pair j); v is a copy of the dv band.
template <int DT>
__global__ __launch_bounds__(256) void qkv_prep_kernel(
    const void* __restrict__ QB, const void* __restrict__ KVB, const void* __restrict__ KR,
    int64_t skr, const float* __restrict__ wqn, const float* __restrict__ wkn,
    const float* __restrict__ cosb, const float* __restrict__ sinb, const int32_t* __restrict__ pos,
    int B, int S, int H, float eps, void* __restrict__ Q, void* __restrict__ DQ,
    void* __restrict__ K, void* __restrict__ DK, void* __restrict__ V, void* __restrict__ DV) {
  constexpr int DN = 32, DR2 = 16, HD = 64, KVW = 96;
  const int row = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
  const int64_t half = (int64_t)B * S;
  if (row >= half) return;
  const int b = __builtin_amdgcn_readfirstlane(row / S);
  const int s = row - b * S;
  const int l = threadIdx.x & 63, hh = l >> 3, c = l & 7;
  const bool nope = c < 4;
  const int sd = pos ? pos[s] : s;
  const uint16_t* qb = static_cast<const uint16_t*>(QB);
  const uint16_t* kvb = static_cast<const uint16_t*>(KVB);
  const uint16_t* kr = static_cast<const uint16_t*>(KR);
  auto ld16 = [](const uint16_t* p, int64_t i) { return *reinterpret_cast<const uint4*>(p + i); };
  auto st16 = [](void* p, int64_t i, const uint4& v) {
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) = v;
  };
  // the rotation factors of this lane's four rope pairs
  float cs[4], sn[4];
  if (!nope) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      cs[j] = cosb[(int64_t)s * DR2 + 4 * (c - 4) + j];
      sn[j] = sinb[(int64_t)s * DR2 + 4 * (c - 4) + j];
    }
  }
  // nope: y = w x / r, dy = w (dx / r - x mean(x dx) / r^3) over the head's 32
  // channels; rope: rotate (x, dx) pairwise
  auto head = [&](const uint4& ux, const uint4& ud, const float* w, void* Y, void* DY,
                  int64_t dst) {
    float x[8], d[8], y[8], dy[8];
    unpack8<DT>(ux, x);
    unpack8<DT>(ud, d);
    float ss = 0.f, sxd = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ss += x[j] * x[j];
      sxd += x[j] * d[j];
    }
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    sxd += __shfl_xor(sxd, 1, 64);
    sxd += __shfl_xor(sxd, 2, 64);
    if (nope) {
      const float inv_r = 1.f / sqrtf(ss / (float)DN + eps);
      const float k3 = (sxd / (float)DN) * inv_r * inv_r * inv_r;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float wj = w[8 * c + j];
        y[j] = wj * x[j] * inv_r;
        dy[j] = wj * (d[j] * inv_r - x[j] * k3);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        y[2 * j] = x[2 * j] * cs[j] - x[2 * j + 1] * sn[j];
        y[2 * j + 1] = x[2 * j] * sn[j] + x[2 * j + 1] * cs[j];
        dy[2 * j] = d[2 * j] * cs[j] - d[2 * j + 1] * sn[j];
        dy[2 * j + 1] = d[2 * j] * sn[j] + d[2 * j + 1] * cs[j];
      }
    }
    st16(Y, dst, pack8<DT>(y));
    st16(DY, dst, pack8<DT>(dy));
  };
  for (int g0 = 0; g0 < H; g0 += 8) {
    const int h = g0 + hh;
    if (h >= H) continue;
    const int64_t dst = (((int64_t)b * H + h) * S + sd) * HD + 8 * c;  // (B,H,L,64) chunk
    const int64_t qo = (int64_t)row * (H * HD) + h * HD + 8 * c;
    head(ld16(qb, qo), ld16(qb, qo + half * (H * HD)), wqn, Q, DQ, dst);
    const int64_t ko = (int64_t)row * (H * KVW) + h * KVW;
    const int64_t kt = half * (H * KVW);
    // k: the head's nope chunks from KVB, the shared rope band from KR
    const uint16_t* kx = nope ? kvb + ko + 8 * c : kr + (int64_t)row * skr + 8 * (c - 4);
    const int64_t kd = nope ? kt : half * skr;
    head(ld16(kx, 0), ld16(kx, kd), wkn, K, DK, dst);
    // v: the dv band (64 channels) of this head, chunk c
    st16(V, dst, ld16(kvb, ko + DN + 8 * c));
    st16(DV, dst, ld16(kvb, ko + kt + DN + 8 * c));
  }
}

// ---------------------------------------------------------------------------
// One wave per token row, heads in groups of 8 as above: lane 8 hh + c owns
// channels 8c..8c+7 of head 8 g + hh; out rows (2BS, H*64) stacked
// [primal; tangent].
template <int DT>
__global__ __launch_bounds__(256) void out_gate_kernel(const float* __restrict__ O,
                                                      const float* __restrict__ DO,
                                                      const int32_t* __restrict__ pos,
                                                      const void* __restrict__ Z, int B, int S,
                                                      int H, void* __restrict__ OUT) {
  const int row = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
  const int64_t half = (int64_t)B * S;
  if (row >= half) return;
  const int b = __builtin_amdgcn_readfirstlane(row / S);
  const int s = row - b * S;
  const int l = threadIdx.x & 63, hh = l >> 3, c = l & 7;
  const int sd = pos ? pos[s] : s;
  const uint16_t* z16 = static_cast<const uint16_t*>(Z);
  uint16_t* o16 = static_cast<uint16_t*>(OUT);
  for (int g0 = 0; g0 < H; g0 += 8) {
    const int h = g0 + hh;
    if (h >= H) continue;
    const int64_t src = (((int64_t)b * H + h) * S + sd) * 64 + 8 * c;
    const int64_t op = (int64_t)row * (H * 64) + h * 64 + 8 * c;
    const int64_t opt = op + half * (H * 64);
    float a[8], da[8];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const float4 u = reinterpret_cast<const float4*>(O + src)[p];
      const float4 du = reinterpret_cast<const float4*>(DO + src)[p];
      // the op's fp32 output is first stored as 16-bit (the reference's attention buffer)
      a[4 * p] = IO<DT>::rt(u.x);
      a[4 * p + 1] = IO<DT>::rt(u.y);
      a[4 * p + 2] = IO<DT>::rt(u.z);
      a[4 * p + 3] = IO<DT>::rt(u.w);
      da[4 * p] = IO<DT>::rt(du.x);
      da[4 * p + 1] = IO<DT>::rt(du.y);
      da[4 * p + 2] = IO<DT>::rt(du.z);
      da[4 * p + 3] = IO<DT>::rt(du.w);
    }
    if (Z != nullptr) {
      float zz[8], dz[8];
      unpack8<DT>(*reinterpret_cast<const uint4*>(z16 + op), zz);
      unpack8<DT>(*reinterpret_cast<const uint4*>(z16 + opt), dz);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sg = sigmoidf_(zz[j]);
        const float ga = a[j] * sg;
        da[j] = da[j] * sg + a[j] * sg * (1.f - sg) * dz[j];
        a[j] = ga;
      }
    }
    *reinterpret_cast<uint4*>(o16 + op) = pack8<DT>(a);
    *reinterpret_cast<uint4*>(o16 + opt) = pack8<DT>(da);
  }
}

// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void situ_jvp_kernel(const void* __restrict__ GU, int64_t rows,
                                                      int F, float beta, void* __restrict__ ACT) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= rows * F) return;
  const int64_t row = idx / F;
  const int c = (int)(idx - row * F);
  const int64_t gp = row * (2 * F) + c, gt = (row + rows) * (2 * F) + c;
  const float g = IO<DT>::ld(GU, gp), u = IO<DT>::ld(GU, gp + F);
  const float dg = IO<DT>::ld(GU, gt), du = IO<DT>::ld(GU, gt + F);
  const float sg = sigmoidf_(g);
  const float th = tanhf(g / beta);
  const float act = beta * th * sg;
  const float dact = (1.f - th * th) * sg + beta * th * sg * (1.f - sg);
  IO<DT>::st(ACT, row * F + c, act * u);
  IO<DT>::st(ACT, (row + rows) * F + c, dact * dg * u + act * du);
}

// Eight consecutive columns per thread with 16-byte accesses (F % 8 == 0 and
// 16-byte aligned buffers); the same arithmetic as situ_jvp_kernel.
template <int DT>
__global__ __launch_bounds__(256) void situ_jvp8_kernel(const void* __restrict__ GU, int64_t rows,
                                                       int F, float beta, void* __restrict__ ACT) {
  using T16 = typename T16Of<DT>::T;
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (idx >= rows * F) return;
  const int64_t row = idx / F;
  const int c = (int)(idx - row * F);
  const uint16_t* gu = static_cast<const uint16_t*>(GU);
  const int64_t gp = row * (2 * F) + c, gt = (row + rows) * (2 * F) + c;
  auto ld8 = [&](int64_t i, float (&x)[8]) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(gu + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = T16::to_f32((uint16_t)(v[e] & 0xffff));
      x[2 * e + 1] = T16::to_f32((uint16_t)(v[e] >> 16));
    }
  };
  float g[8], u[8], dg[8], du[8], h[8], dh[8];
  ld8(gp, g);
  ld8(gp + F, u);
  ld8(gt, dg);
  ld8(gt + F, du);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float sg = sigmoidf_(g[e]);
    const float th = tanhf(g[e] / beta);
    const float act = beta * th * sg;
    const float dact = (1.f - th * th) * sg + beta * th * sg * (1.f - sg);
    h[e] = act * u[e];
    dh[e] = dact * dg[e] * u[e] + act * du[e];
  }
  u32x4 hv, dv;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hv[e] = pack_pair<T16>(h[2 * e], h[2 * e + 1]);
    dv[e] = pack_pair<T16>(dh[2 * e], dh[2 * e + 1]);
  }
  uint16_t* out = static_cast<uint16_t*>(ACT);
  *reinterpret_cast<u32x4*>(out + row * F + c) = hv;
  *reinterpret_cast<u32x4*>(out + (row + rows) * F + c) = dv;
}

template <int TI, int TO>
static void launch_rms(const void* x, const void* dx, const float* w, int64_t rows, int D,
                       int64_t sx, void* y, void* dy, int64_t sy, float eps, hipStream_t st) {
  const unsigned grid = (unsigned)((rows + 3) / 4);
  if (D <= 256)
    rmsnorm_jvp_kernel<TI, TO, 4><<<grid, 256, 0, st>>>(x, dx, w, rows, D, sx, y, dy, sy, eps);
  else if (D <= 512)
    rmsnorm_jvp_kernel<TI, TO, 8><<<grid, 256, 0, st>>>(x, dx, w, rows, D, sx, y, dy, sy, eps);
  else
    rmsnorm_jvp_kernel<TI, TO, 16><<<grid, 256, 0, st>>>(x, dx, w, rows, D, sx, y, dy, sy, eps);
}

}  // namespace

}  // namespace sla2h

using namespace sla2h;

extern "C" int sla2h_rmsnorm_jvp(const void* x, const void* dx, int in_dtype, const float* w,
                                 int64_t rows, int D, int64_t sx, void* y, void* dy, int64_t sy,
                                 int out_dtype, float eps, void* stream) {
  SLA2H_CHECK_ARG(x && dx && w && y && dy);
  SLA2H_CHECK_ARG(rows > 0 && D > 0 && D <= 1024 && sx >= D && sy >= D);
  SLA2H_CHECK_ARG(in_dtype >= 0 && in_dtype <= 2 && out_dtype >= 0 && out_dtype <= 2);
  SLA2H_CHECK_ARG((rows + 3) / 4 < (1ll << 31));
  hipStream_t st = static_cast<hipStream_t>(stream);
  // in: fp32 (the residual stream) or 16-bit (GEMM outputs); out: 16-bit or fp32
#define SLA2H_RMS(TI, TO) launch_rms<TI, TO>(x, dx, w, rows, D, sx, y, dy, sy, eps, st)
  if (in_dtype == kF32 && out_dtype == SLA2H_DTYPE_F16) SLA2H_RMS(kF32, SLA2H_DTYPE_F16);
  else if (in_dtype == kF32 && out_dtype == SLA2H_DTYPE_BF16) SLA2H_RMS(kF32, SLA2H_DTYPE_BF16);
  else if (in_dtype == kF32 && out_dtype == kF32) SLA2H_RMS(kF32, kF32);
  else if (in_dtype == SLA2H_DTYPE_F16 && out_dtype == SLA2H_DTYPE_F16) SLA2H_RMS(SLA2H_DTYPE_F16, SLA2H_DTYPE_F16);
  else if (in_dtype == SLA2H_DTYPE_BF16 && out_dtype == SLA2H_DTYPE_BF16) SLA2H_RMS(SLA2H_DTYPE_BF16, SLA2H_DTYPE_BF16);
  else return (int)hipErrorInvalidValue;
#undef SLA2H_RMS
  return (int)hipGetLastError();
}

extern "C" int sla2h_mla_qkv_prep(const void* qb, const void* kvb, const void* kr, int64_t skr,
                                  const float* w_qnorm, const float* w_knorm, const float* rope_cos,
                                  const float* rope_sin, const int32_t* pos, int dtype, int B,
                                  int S, int H, int dn, int dr, int dv, float eps, void* q,
                                  void* dq, void* k, void* dk, void* v, void* dv_out,
                                  void* stream) {
  SLA2H_CHECK_ARG(qb && kvb && kr && w_qnorm && w_knorm && rope_cos && rope_sin);
  SLA2H_CHECK_ARG(q && dq && k && dk && v && dv_out);
  SLA2H_CHECK_ARG(dn == 32 && dr == 32 && dv == 64 && skr >= dr);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && S > 0 && H > 0);
  // 16-byte chunks: row strides a multiple of 8 elements, 16-byte aligned bases
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  SLA2H_CHECK_ARG(skr % 8 == 0 && al16(qb) && al16(kvb) && al16(kr) && al16(q) && al16(dq) &&
                  al16(k) && al16(dk) && al16(v) && al16(dv_out));
  const int64_t units = (int64_t)B * S;  // one wave per token row
  SLA2H_CHECK_ARG(units + 3 < (1ll << 31));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned grid = (unsigned)((units + 3) / 4);
  if (dtype == SLA2H_DTYPE_F16)
    qkv_prep_kernel<SLA2H_DTYPE_F16><<<grid, 256, 0, st>>>(qb, kvb, kr, skr, w_qnorm, w_knorm, rope_cos, rope_sin, pos, B, S, H, eps, q, dq, k, dk, v, dv_out);
  else
    qkv_prep_kernel<SLA2H_DTYPE_BF16><<<grid, 256, 0, st>>>(qb, kvb, kr, skr, w_qnorm, w_knorm, rope_cos, rope_sin, pos, B, S, H, eps, q, dq, k, dk, v, dv_out);
  return (int)hipGetLastError();
}

extern "C" int sla2h_mla_out_gate(const float* o, const float* dout, const int32_t* pos,
                                  const void* z, int dtype, int B, int S, int H, int dv,
                                  void* out, void* stream) {
  SLA2H_CHECK_ARG(o && dout && out);
  SLA2H_CHECK_ARG(dv == 64 && B > 0 && S > 0 && H > 0);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  const int64_t units = (int64_t)B * S;  // one wave per token row
  SLA2H_CHECK_ARG(units + 3 < (1ll << 31));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned grid = (unsigned)((units + 3) / 4);
  if (dtype == SLA2H_DTYPE_F16)
    out_gate_kernel<SLA2H_DTYPE_F16><<<grid, 256, 0, st>>>(o, dout, pos, z, B, S, H, out);
  else
    out_gate_kernel<SLA2H_DTYPE_BF16><<<grid, 256, 0, st>>>(o, dout, pos, z, B, S, H, out);
  return (int)hipGetLastError();
}

extern "C" int sla2h_situ_jvp(const void* gu, int64_t rows, int F, float beta, int dtype,
                              void* act, void* stream) {
  SLA2H_CHECK_ARG(gu && act && rows > 0 && F > 0 && beta > 0.f);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  const int64_t n = rows * F;
  SLA2H_CHECK_ARG((n + 255) / 256 < (1ll << 31));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (F % 8 == 0 && reinterpret_cast<uintptr_t>(gu) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(act) % 16 == 0) {
    const unsigned grid8 = (unsigned)((n / 8 + 255) / 256);
    if (dtype == SLA2H_DTYPE_F16)
      situ_jvp8_kernel<SLA2H_DTYPE_F16><<<grid8, 256, 0, st>>>(gu, rows, F, beta, act);
    else
      situ_jvp8_kernel<SLA2H_DTYPE_BF16><<<grid8, 256, 0, st>>>(gu, rows, F, beta, act);
    return (int)hipGetLastError();
  }
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (dtype == SLA2H_DTYPE_F16)
    situ_jvp_kernel<SLA2H_DTYPE_F16><<<grid, 256, 0, st>>>(gu, rows, F, beta, act);
  else
    situ_jvp_kernel<SLA2H_DTYPE_BF16><<<grid, 256, 0, st>>>(gu, rows, F, beta, act);
  return (int)hipGetLastError();
}
