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
// One wave per (token row, head); dn = dr = 32, dv = 64 (qk head dim 64).
// Lane l: nope channel pair (l & 15) * 2 .. +1 for the query (lanes 0-15),
// the key (lanes 16-31); rope pair i = l & 15 for the query (lanes 32-47) and
// the key (lanes 48-63).  v: every lane copies one channel.
template <int DT>
__global__ __launch_bounds__(256) void qkv_prep_kernel(
    const void* __restrict__ QB, const void* __restrict__ KVB, const void* __restrict__ KR,
    int64_t skr, const float* __restrict__ wqn, const float* __restrict__ wkn,
    const float* __restrict__ cosb, const float* __restrict__ sinb, const int32_t* __restrict__ pos,
    int B, int S, int H, float eps, void* __restrict__ Q, void* __restrict__ DQ,
    void* __restrict__ K, void* __restrict__ DK, void* __restrict__ V, void* __restrict__ DV) {
  constexpr int DN = 32, DR2 = 16, HD = 64, DVW = 64;
  // (row, head) of this wave, uniform: 32-bit index math pinned to SGPRs
  const int unit = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
  const int64_t half = (int64_t)B * S;
  if (unit >= half * H) return;
  const int h = __builtin_amdgcn_readfirstlane(unit % H);
  const int row = __builtin_amdgcn_readfirstlane(unit / H);  // primal token row b*S + s
  const int b = __builtin_amdgcn_readfirstlane(row / S);
  const int s = row - b * S;
  const int l = threadIdx.x & 63;
  const int i = l & 15;
  const int64_t dst = (((int64_t)b * H + h) * S + (pos ? pos[s] : s)) * HD;  // (B,H,L,64) row
  const int64_t qrow = row * (H * HD), qrow_t = (row + half) * (H * HD);
  const int64_t kvw = DN + DVW;
  const int64_t krow = row * (H * kvw), krow_t = (row + half) * (H * kvw);
  const int sel = l >> 4;  // 0 q nope, 1 k nope, 2 q rope, 3 k rope
  if (sel < 2) {
    const void* src = sel == 0 ? QB : KVB;
    const int64_t base = sel == 0 ? qrow + h * HD : krow + h * kvw;
    const int64_t base_t = sel == 0 ? qrow_t + h * HD : krow_t + h * kvw;
    const float2 xx = IO<DT>::ld2(src, base + 2 * i), dd = IO<DT>::ld2(src, base_t + 2 * i);
    const float x0 = xx.x, x1 = xx.y, d0 = dd.x, d1 = dd.y;
    const float ss = sum16(x0 * x0 + x1 * x1);
    const float sxd = sum16(x0 * d0 + x1 * d1);
    const float inv_r = 1.f / sqrtf(ss / (float)DN + eps);
    const float k3 = (sxd / (float)DN) * inv_r * inv_r * inv_r;
    const float* w = sel == 0 ? wqn : wkn;
    void* Y = sel == 0 ? Q : K;
    void* DY = sel == 0 ? DQ : DK;
    IO<DT>::st2(Y, dst + 2 * i, w[2 * i] * x0 * inv_r, w[2 * i + 1] * x1 * inv_r);
    IO<DT>::st2(DY, dst + 2 * i, w[2 * i] * (d0 * inv_r - x0 * k3),
                w[2 * i + 1] * (d1 * inv_r - x1 * k3));
  } else {
    const float c = cosb[(int64_t)s * DR2 + i], sn = sinb[(int64_t)s * DR2 + i];
    float xr, xi, dr_, di;
    float2 xx, dd;
    if (sel == 2) {
      xx = IO<DT>::ld2(QB, qrow + h * HD + DN + 2 * i);
      dd = IO<DT>::ld2(QB, qrow_t + h * HD + DN + 2 * i);
    } else {
      xx = IO<DT>::ld2(KR, row * skr + 2 * i);
      dd = IO<DT>::ld2(KR, (row + half) * skr + 2 * i);
    }
    xr = xx.x;
    xi = xx.y;
    dr_ = dd.x;
    di = dd.y;
    void* Y = sel == 2 ? Q : K;
    void* DY = sel == 2 ? DQ : DK;
    IO<DT>::st2(Y, dst + DN + 2 * i, xr * c - xi * sn, xr * sn + xi * c);
    IO<DT>::st2(DY, dst + DN + 2 * i, dr_ * c - di * sn, dr_ * sn + di * c);
  }
  // v: straight copy of the dv band (lane l = channel l)
  IO<DT>::st(V, dst + l, IO<DT>::ld(KVB, krow + h * kvw + DN + l));
  IO<DT>::st(DV, dst + l, IO<DT>::ld(KVB, krow_t + h * kvw + DN + l));
}

// ---------------------------------------------------------------------------
// One wave per (token row, head): out rows (2BS, H*64) stacked [primal; tangent].
template <int DT>
__global__ __launch_bounds__(256) void out_gate_kernel(const float* __restrict__ O,
                                                      const float* __restrict__ DO,
                                                      const int32_t* __restrict__ pos,
                                                      const void* __restrict__ Z, int B, int S,
                                                      int H, void* __restrict__ OUT) {
  const int unit = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
  const int64_t half = (int64_t)B * S;
  if (unit >= half * H) return;
  const int h = __builtin_amdgcn_readfirstlane(unit % H);
  const int64_t row = __builtin_amdgcn_readfirstlane(unit / H);
  const int b = __builtin_amdgcn_readfirstlane((int)row / S);
  const int s = (int)row - b * S;
  const int l = threadIdx.x & 63;
  const int64_t src = (((int64_t)b * H + h) * S + (pos ? pos[s] : s)) * 64 + l;
  // the op's fp32 output is first stored as 16-bit (the reference's attention buffer)
  const float a = IO<DT>::rt(O[src]), da = IO<DT>::rt(DO[src]);
  const int64_t op = row * (H * 64) + h * 64 + l, opt = (row + half) * (H * 64) + h * 64 + l;
  if (Z == nullptr) {
    IO<DT>::st(OUT, op, a);
    IO<DT>::st(OUT, opt, da);
    return;
  }
  const float z = IO<DT>::ld(Z, op), dz = IO<DT>::ld(Z, opt);
  const float sg = sigmoidf_(z);
  IO<DT>::st(OUT, op, a * sg);
  IO<DT>::st(OUT, opt, da * sg + a * sg * (1.f - sg) * dz);
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
  // channel pairs move as 32-bit words: even strides, 4-byte aligned rows
  auto al4 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3) == 0; };
  SLA2H_CHECK_ARG(skr % 2 == 0 && al4(qb) && al4(kvb) && al4(kr) && al4(q) && al4(dq) &&
                  al4(k) && al4(dk));
  const int64_t units = (int64_t)B * S * H;
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
  const int64_t units = (int64_t)B * S * H;
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
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (dtype == SLA2H_DTYPE_F16)
    situ_jvp_kernel<SLA2H_DTYPE_F16><<<grid, 256, 0, st>>>(gu, rows, F, beta, act);
  else
    situ_jvp_kernel<SLA2H_DTYPE_BF16><<<grid, 256, 0, st>>>(gu, rows, F, beta, act);
  return (int)hipGetLastError();
}
