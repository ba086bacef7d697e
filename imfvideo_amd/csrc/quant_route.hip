// INT8 block quantisation, router tile pooling and block top-k for gfx950.
//
// This translation unit is compiled with -ffp-contract=off: every fp32
// product and sum below rounds separately, in the order written, so the
// results are bit-identical to the CPU restatement in oracle/.
//
// Reference semantics:
//   quantisation  models/sla2_vendor/kernel_sparse_qat.py:120-151
//   tile pooling  models/mla_video_sparse_jvp.py:506-529, 545-562
//   scores+top-k  models/mla_video_sparse_jvp.py:563-565, 292-294
#include "common.h"

#include <type_traits>

namespace sla2h {

constexpr int kTile = 64;  // E = D = 64

struct QuantPoolArgs {
  const uint16_t* x[2];   // (BH, L, 64) 16-bit
  int8_t* xq[2];          // (BH, L, 64)
  float* xs[2];           // (BH, Nb)
  float* pool[2];         // q: (BH, Nb, 64); k: (BH, 64, npool) transposed; may be null
  const float* proj[2];   // (64, 64) or null
  int npool[2];           // number of leading blocks to pool
  int64_t pool_len[2];    // rows that count for pooling (L for q, Np*E for k)
  int transposed[2];
  float* kb[2];           // (BH, Nb) or null: bound on the tile's dequantised row norms
  int BH;
  int64_t L;
  int Nb;
};

// Exact quotient fl(x / s) without a division per element (Markstein's
// correction): with r = fl(1 / s) correctly rounded and q0 = fl(x r) within an
// ulp of x / s, e = x - q0 s is exact under the FMA and fl(q0 + e r) is the
// correctly rounded quotient (checked against IEEE division for every 16-bit
// x and tile maximum: equal except for denormal x, whose quotients both
// round to 0).
__device__ inline float quotient(float x, float s, float r) {
  const float q0 = x * r;
  return __builtin_fmaf(__builtin_fmaf(-q0, s, x), r, q0);
}

// Round half away from zero of the quotient q = quotient(x, s, 1/s):
// trunc(fl(q + sign(x) (0.5 - 2^-25))).  The constant just below 0.5 keeps
// q = 0.5 - 2^-25 at 0 (q + 0.5 would round up to 1 there), and exact ties
// k + 0.5 still round away (the sum rounds up to k + 1).  With x and the tile
// maximum both 16-bit values this equals (int)roundf(fl(x / s)) for every
// pair (exhaustive check: tests/quant_law_check.c).
__device__ inline int round_away(float q, float x) {
  return (int)(q + __builtin_copysignf(0x1.fffffep-2f, x));
}
// Low bytes of four int32 values packed into one word (three v_perm_b32)
__device__ inline uint32_t pack_bytes(int b0, int b1, int b2, int b3) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)b1, (uint32_t)b0, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)b3, (uint32_t)b2, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// Tiles are numbered i = (tensor * BH + bh) * Nb + blk.  Each workgroup of 256
// threads takes tiles i = blockIdx.x, + G, ... (G = gridDim.x) and keeps the
// loads of the next kQuantSets - 1 tiles in flight while it quantises the
// current one: kQuantSets register sets, each reloaded with the tile
// kQuantSets G further on as soon as its data is consumed (the loop is
// unrolled over the sets, so no set is ever copied -- a register copy would
// wait for its load).  Thread tid owns row tid / 4, channels 16 (tid % 4) ..
// +15.  The pooling sums run in wave 0 from a double-buffered LDS copy of the
// tile, so one barrier per tile.
constexpr int kQuantSets = 3;

template <typename T16>
__global__ __launch_bounds__(256) void quant_pool_kernel(QuantPoolArgs a, int ntiles) {
  __shared__ __align__(16) uint16_t tile[2][kTile][kTile];
  __shared__ float red[2][4];
  __shared__ float rnorm[2][4];
  __shared__ float vec[2][kTile];

  const int tid = threadIdx.x;
  const int r = tid >> 2;
  const int c0 = (tid & 3) * 16;
  const int G = gridDim.x;
  auto load = [&](int i, uint4 (&u)[2]) {
    if (i >= ntiles) return;
    const int blk = i % a.Nb;
    const int y = i / a.Nb;
    const int t = y / a.BH, bh = y - t * a.BH;
    const int64_t row = (int64_t)blk * kTile + r;
    if (row < a.L) {
      const uint4* src = reinterpret_cast<const uint4*>(a.x[t] + ((int64_t)bh * a.L + row) * kTile + c0);
      u[0] = src[0];
      u[1] = src[1];
    } else {
      u[0] = u[1] = make_uint4(0, 0, 0, 0);
    }
  };
  int buf = 0;
  auto body = [&](int i, uint4 (&u)[2]) {
    const int blk = i % a.Nb;
    const int y = i / a.Nb;
    const int t = y / a.BH, bh = y - t * a.BH;
    const int64_t row = (int64_t)blk * kTile + r;

    const uint32_t wv[8] = {u[0].x, u[0].y, u[0].z, u[0].w, u[1].x, u[1].y, u[1].z, u[1].w};
    float xv[16];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      xv[2 * k] = T16::to_f32((uint16_t)(wv[k] & 0xffff));
      xv[2 * k + 1] = T16::to_f32((uint16_t)(wv[k] >> 16));
    }
    // tile absmax (max is order-independent, so any reduction tree is exact)
    float am = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) am = fmaxf(am, fabsf(xv[k]));
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) am = fmaxf(am, __shfl_xor(am, m, 64));
    if ((tid & 63) == 0) red[buf][tid >> 6] = am;
    // largest squared row norm of the tile (the bound below needs no exact
    // sum: rounding only moves a softmax shift)
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) ss = __builtin_fmaf(xv[k], xv[k], ss);
    ss = ss + __shfl_xor(ss, 1, 64);
    ss = ss + __shfl_xor(ss, 2, 64);
#pragma unroll
    for (int m = 4; m <= 32; m <<= 1) ss = fmaxf(ss, __shfl_xor(ss, m, 64));
    if ((tid & 63) == 0) rnorm[buf][tid >> 6] = ss;
    const bool pooled = a.pool[t] != nullptr && blk < a.npool[t];
    if (pooled) {
      *reinterpret_cast<uint4*>(&tile[buf][r][c0]) = u[0];
      *reinterpret_cast<uint4*>(&tile[buf][r][c0 + 8]) = u[1];
    }
    load(i + kQuantSets * G, u);  // this set's data is consumed: refill it
    __syncthreads();
    am = fmaxf(fmaxf(red[buf][0], red[buf][1]), fmaxf(red[buf][2], red[buf][3]));
    const float s = am / 127.0f + 1e-12f;  // IEEE division, then add
    const float rs = 1.0f / s;             // correctly rounded reciprocal

    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      int qv[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float x = xv[4 * k + b];
        qv[b] = round_away(quotient(x, s, rs), x);
      }
      w[k] = pack_bytes(qv[0], qv[1], qv[2], qv[3]);
    }
    if (row < a.L)
      *reinterpret_cast<uint4*>(a.xq[t] + ((int64_t)bh * a.L + row) * kTile + c0) =
          make_uint4(w[0], w[1], w[2], w[3]);
    if (tid == 0) a.xs[t][(int64_t)bh * a.Nb + blk] = s;
    // kb >= max_j ||x8_j|| s over the tile's rows: each element of x8 s is
    // within s / 2 of x, so ||x8_j s - x_j|| <= 4 s over 64 channels
    if (tid == 0 && a.kb[t] != nullptr) {
      const float mx = fmaxf(fmaxf(rnorm[buf][0], rnorm[buf][1]), fmaxf(rnorm[buf][2], rnorm[buf][3]));
      a.kb[t][(int64_t)bh * a.Nb + blk] = __builtin_sqrtf(mx) * 1.000001f + 4.f * s;
    }

    // ---- pooling (wave 0): sequential per-channel fp32 sum over the real rows ----
    if (pooled && tid < kTile) {
      const int64_t rem = a.pool_len[t] - (int64_t)blk * kTile;
      const int cnt = rem < kTile ? (int)rem : kTile;
      float acc = 0.f;
      int rr = 0;
      for (; rr + 16 <= cnt; rr += 16) {  // 16 LDS reads in flight, then the adds in row order
        float xr[16];
#pragma unroll
        for (int uu = 0; uu < 16; ++uu) xr[uu] = T16::to_f32(tile[buf][rr + uu][tid]);
#pragma unroll
        for (int uu = 0; uu < 16; ++uu) acc = acc + xr[uu];
      }
      for (; rr < cnt; ++rr) acc = acc + T16::to_f32(tile[buf][rr][tid]);
      const float mean = acc / (float)cnt;
      float outv = mean;
      if (a.proj[t] != nullptr) {
        vec[buf][tid] = mean;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        const float* pr = a.proj[t] + tid * kTile;  // row e of proj: out[e] = sum_d x[d] P[e,d]
        float p = 0.f;
        for (int d = 0; d < kTile; ++d) p = p + vec[buf][d] * pr[d];
        outv = p;
      }
      if (a.transposed[t])
        a.pool[t][((int64_t)bh * kTile + tid) * a.npool[t] + blk] = outv;
      else
        a.pool[t][((int64_t)bh * a.Nb + blk) * kTile + tid] = outv;
    }
    buf ^= 1;
  };
  uint4 u0[2], u1[2], u2[2];
  static_assert(kQuantSets == 3, "one register set per unrolled body below");
  const int i0 = blockIdx.x;
  load(i0, u0);
  load(i0 + G, u1);
  load(i0 + 2 * G, u2);
  for (int i = i0; i < ntiles; i += 3 * G) {
    body(i, u0);
    if (i + G >= ntiles) break;
    body(i + G, u1);
    if (i + 2 * G >= ntiles) break;
    body(i + 2 * G, u2);
  }
}

// Training-forward quantisation (semantics of the in-kernel quantisation of
// _attn_fwd_qat, models/sla2_vendor/kernel_sparse_qat.py:56-58, 88-90,
// 106-107): s = max|x| / 127 + 1e-12 per 64 x 64 tile, q = (int) fl(fl(x / s)
// + 0.5 sign(x)) truncated toward zero (sign(+-0) = +1).  Q and K keep the
// row-major (BH, L, 64) int8 layout; V is written as INT8 MFMA A-operand
// fragments of O^T = V8^T P8^T: per tile [ct][lane][16 B], byte s of lane
// (g, rr) of column tile ct = V8[16 (s >> 2) + 4 g + (s & 3)][16 ct + rr].
struct QuantTrainArgs {
  const uint16_t* x[3];  // q, k, v (BH, L, 64)
  int8_t* xq[3];         // q8, k8 (BH, L, 64); v8f (BH, Nb, 4096)
  float* xs[3];          // (BH, Nb)
  int BH;
  int64_t L;
  int Nb;
  int t0;                // first tensor of the grid (blockIdx.y / BH counts from it)
};

// RND: the round-half-away law of quantize_qkv instead (the inference INT8
// path, sla2h_quantize_v8f).
template <typename T16, bool RND = false>
__global__ __launch_bounds__(256) void quant_train_kernel(QuantTrainArgs a) {
  __shared__ float red[4];
  __shared__ __align__(16) int8_t q8t[kTile][kTile + 16];

  const int tid = threadIdx.x;
  const int blk = blockIdx.x;
  const int t = a.t0 + blockIdx.y / a.BH;
  const int bh = blockIdx.y % a.BH;
  const int r = tid >> 2;
  const int c0 = (tid & 3) * 16;
  const int64_t row = (int64_t)blk * kTile + r;
  const bool valid = row < a.L;
  const int64_t off = ((int64_t)bh * a.L + row) * kTile + c0;

  float xv[16];
  if (valid) {
    const uint4* src = reinterpret_cast<const uint4*>(a.x[t] + off);
    uint4 u0 = src[0], u1 = src[1];
    uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      xv[2 * i] = T16::to_f32((uint16_t)(w[i] & 0xffff));
      xv[2 * i + 1] = T16::to_f32((uint16_t)(w[i] >> 16));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) xv[i] = 0.f;
  }
  float am = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) am = fmaxf(am, fabsf(xv[i]));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) am = fmaxf(am, __shfl_xor(am, m, 64));
  if ((tid & 63) == 0) red[tid >> 6] = am;
  __syncthreads();
  am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = am / 127.0f + 1e-12f;

  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t acc = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float x = xv[4 * i + b];
      int qv;
      if (RND) {
        qv = (int)roundf(x / s);  // round half away from zero
      } else {
        const float y = x / s + (x >= 0.f ? 0.5f : -0.5f);  // two roundings (no contraction)
        qv = (int)y;
      }
      acc |= ((uint32_t)(qv & 0xff)) << (8 * b);
    }
    w[i] = acc;
  }
  if (tid == 0) a.xs[t][(int64_t)bh * a.Nb + blk] = s;
  if (t < 2) {
    if (valid) *reinterpret_cast<uint4*>(a.xq[t] + off) = make_uint4(w[0], w[1], w[2], w[3]);
    return;
  }
  // V: transpose to the fragment order through LDS (rows past L are zero)
  *reinterpret_cast<uint4*>(&q8t[r][c0]) = make_uint4(w[0], w[1], w[2], w[3]);
  __syncthreads();
  const int ct = tid >> 6, lane = tid & 63, g = lane >> 4, rr = lane & 15;
  uint32_t f[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc |= ((uint32_t)(uint8_t)q8t[16 * kb + 4 * g + i][16 * ct + rr]) << (8 * i);
    f[kb] = acc;
  }
  *reinterpret_cast<uint4*>(a.xq[2] + ((int64_t)bh * a.Nb + blk) * 4096 + tid * 16) =
      make_uint4(f[0], f[1], f[2], f[3]);
}

// quantize_qkv / _quant_blocks (models/sla2_vendor/kernel_sparse_qat.py:
// 120-151) for blocks of E = 32..256 rows: one block per workgroup, thread t
// holds E/4 consecutive elements (a segment of one row), s = max|x| / 127 +
// 1e-12, q = round half away from zero of x / s.  TRUNC: the training
// kernel's law instead, q = (int) fl(fl(x / s) + 0.5 sign(x)) (the in-kernel
// Q quantisation of _attn_fwd_qat, kernel_sparse_qat.py:56-58, for BLOCK_M =
// bq rows).
template <typename T16, int E, bool TRUNC = false>
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* __restrict__ x, int64_t L,
                                                         int Nb, int8_t* __restrict__ xq,
                                                         float* __restrict__ xs) {
  constexpr int PER = E / 4;
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int blk = blockIdx.x;
  const int bh = blockIdx.y;
  const int e0 = tid * PER;
  const bool valid = (int64_t)blk * E + e0 / kTile < L;
  const int64_t off = ((int64_t)bh * L + (int64_t)blk * E) * kTile + e0;
  float xv[PER];
#pragma unroll
  for (int c = 0; c < PER / 8; ++c) {
    const uint4 u = valid ? reinterpret_cast<const uint4*>(x + off)[c] : make_uint4(0, 0, 0, 0);
    const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xv[8 * c + 2 * i] = T16::to_f32((uint16_t)(wd[i] & 0xffff));
      xv[8 * c + 2 * i + 1] = T16::to_f32((uint16_t)(wd[i] >> 16));
    }
  }
  float am = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) am = fmaxf(am, fabsf(xv[i]));
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) am = fmaxf(am, __shfl_xor(am, m, 64));
  if ((tid & 63) == 0) red[tid >> 6] = am;
  __syncthreads();
  am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = am / 127.0f + 1e-12f;  // IEEE division, then add
  uint32_t w[PER / 4];
#pragma unroll
  for (int i = 0; i < PER / 4; ++i) {
    uint32_t acc = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float xx = xv[4 * i + b];
      const int qv = TRUNC ? (int)(xx / s + (xx >= 0.f ? 0.5f : -0.5f)) : (int)roundf(xx / s);
      acc |= ((uint32_t)(qv & 0xff)) << (8 * b);
    }
    w[i] = acc;
  }
  if (valid) {
    if (PER == 8) {
      *reinterpret_cast<uint2*>(xq + off) = make_uint2(w[0], w[1]);
    } else {
#pragma unroll
      for (int c = 0; c < PER / 16; ++c)
        reinterpret_cast<uint4*>(xq + off)[c] =
            make_uint4(w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]);
    }
  }
  if (tid == 0) xs[(int64_t)bh * Nb + blk] = s;
}

// Orderable 64-bit key: high word = monotone map of the fp32 score
// (NaN -> +NaN, the largest, as torch.topk orders; -0 -> +0), low word =
// ~index so that equal scores rank the lower index first.
__device__ inline uint64_t score_key(float sc, int n) {
  uint32_t u = __builtin_bit_cast(uint32_t, sc);
  if (sc != sc) u = 0x7fc00000u;
  if (u == 0x80000000u) u = 0u;
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - (uint32_t)n);
}

// ROWS query blocks of one (b,h) per workgroup: scores into LDS, one
// bitonic sort (descending) per row over P2 = next_pow2(Np) keys, emit top T.
template <int ROWS>
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ qpool,
                                                         const float* __restrict__ kpool_t,
                                                         int Mb, int Np, int T, float scale,
                                                         int P2, int32_t* __restrict__ lut,
                                                         uint8_t* __restrict__ mask) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* keys = reinterpret_cast<uint64_t*>(smem);                 // ROWS * P2
  float* qsh = reinterpret_cast<float*>(smem + (size_t)ROWS * P2 * 8);  // ROWS * 64
  uint8_t* sel = smem + (size_t)ROWS * P2 * 8 + ROWS * kTile * 4;      // ROWS * P2

  const int tid = threadIdx.x;
  const int bh = blockIdx.y;
  const int m0 = blockIdx.x * ROWS;

  for (int idx = tid; idx < ROWS * kTile; idx += 256) {
    const int rr = idx / kTile, d = idx % kTile;
    const int m = m0 + rr;
    qsh[idx] = (m < Mb) ? qpool[((int64_t)bh * Mb + m) * kTile + d] : 0.f;
  }
  for (int idx = tid; idx < ROWS * P2; idx += 256) sel[idx] = 0;
  __syncthreads();

  const float* kt = kpool_t + (int64_t)bh * kTile * Np;
  for (int n = tid; n < P2; n += 256) {
    if (n < Np) {
      float acc[ROWS];
#pragma unroll
      for (int rr = 0; rr < ROWS; ++rr) acc[rr] = 0.f;
      for (int d = 0; d < kTile; ++d) {
        const float kv = kt[(int64_t)d * Np + n];
#pragma unroll
        for (int rr = 0; rr < ROWS; ++rr) acc[rr] = acc[rr] + qsh[rr * kTile + d] * kv;
      }
#pragma unroll
      for (int rr = 0; rr < ROWS; ++rr) keys[rr * P2 + n] = score_key(acc[rr] * scale, n);
    } else {
#pragma unroll
      for (int rr = 0; rr < ROWS; ++rr) keys[rr * P2 + n] = 0ull;  // below every real key
    }
  }
  __syncthreads();

  const int half = P2 >> 1;
  for (int k = 2; k <= P2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int idx = tid; idx < ROWS * half; idx += 256) {
        const int rr = idx / half, h = idx % half;
        const int i = (h / j) * 2 * j + (h % j);
        const int l = i + j;
        uint64_t* row = keys + rr * P2;
        const uint64_t ki = row[i], kl = row[l];
        const bool desc = (i & k) == 0;  // overall order: descending
        if (desc ? (ki < kl) : (ki > kl)) {
          row[i] = kl;
          row[l] = ki;
        }
      }
      __syncthreads();
    }
  }

  for (int idx = tid; idx < ROWS * T; idx += 256) {
    const int rr = idx / T, jj = idx % T;
    const int m = m0 + rr;
    const uint32_t n = 0xffffffffu - (uint32_t)(keys[rr * P2 + jj] & 0xffffffffull);
    if (m < Mb) lut[((int64_t)bh * Mb + m) * T + jj] = (int32_t)n;
    sel[rr * P2 + n] = 1;
  }
  if (mask == nullptr) return;
  __syncthreads();
  for (int idx = tid; idx < ROWS * Np; idx += 256) {
    const int rr = idx / Np, n = idx % Np;
    const int m = m0 + rr;
    if (m < Mb) mask[((int64_t)bh * Mb + m) * Np + n] = sel[rr * P2 + n];
  }
}

// Top-T of each row by wave-wide radix selection (T <= 64): one wave per
// query block, NK keys per lane (tile n = lane + 64 i), R rows per wave.
//   1. scores, same sequential fp32 order as route_topk_kernel;
//   2. s* = the T-th largest order-preserving score word (32-bit binary
//      search with ballot counts); if several keys share s*, the lowest
//      indices among them fill up to T (a 12-bit binary search over n);
//   3. the T winners are compacted through LDS and bitonic-sorted across
//      the lanes by their 64-bit keys (score word, then lower index first).
template <int NK, int R, bool V4>
__global__ __launch_bounds__(256) void route_select_kernel(const float* __restrict__ qpool,
                                                           const float* __restrict__ kpool_t,
                                                           int Mb, int Np, int T, float scale,
                                                           int32_t* __restrict__ lut,
                                                           uint8_t* __restrict__ mask) {
  // pooled keys of the head, staged in chunks of DC channels (32 KB) that the
  // four waves share
  constexpr int DC = 128 / NK;
  __shared__ float ksh[DC][64 * NK];
  __shared__ uint64_t win[4][64];
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int bh = blockIdx.y;
  const int m0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + w) * R);
  const bool active = m0 < Mb;  // uniform per wave; every wave takes the barriers

  const float* kt = kpool_t + (int64_t)bh * kTile * Np;
  float acc[R][NK];
#pragma unroll
  for (int rr = 0; rr < R; ++rr)
#pragma unroll
    for (int i = 0; i < NK; ++i) acc[rr][i] = 0.f;
  // lane d holds q[row][d] (broadcast with readlane).  Key slots past Np
  // need no guard: their scores are never selected (ord = 0 below); the
  // buffer range check returns 0 past the end of this head's pooled keys.
  const float* qrow = qpool + ((int64_t)bh * Mb + m0) * kTile;
  float qlane[R];
#pragma unroll
  for (int rr = 0; rr < R; ++rr) qlane[rr] = (m0 + rr < Mb) ? qrow[rr * kTile + lane] : 0.f;
  const auto rk = make_rsrc(kt, (int64_t)kTile * Np * 4);
  for (int d0 = 0; d0 < kTile; d0 += DC) {
    __syncthreads();  // the previous chunk is consumed
    if constexpr (V4) {
      // Np % 4 == 0: a channel's row of Np floats is 16-byte aligned, so one
      // 16-byte load carries 4 keys (a load at n < Np lies inside the row)
#pragma unroll
      for (int k = 0; k < DC * 16 * NK / 256; ++k) {
        const int e = tid + 256 * k;
        const int dd = e / (16 * NK), n = 4 * (e % (16 * NK));
        *reinterpret_cast<u32x4*>(&ksh[dd][n]) = buf_load16(rk, ((d0 + dd) * Np + n) * 4, 0);
      }
    } else {
#pragma unroll
      for (int k = 0; k < DC * 64 * NK / 256; ++k) {
        const int e = tid + 256 * k;
        const int dd = e / (64 * NK), n = e % (64 * NK);
        ksh[dd][n] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                   rk, ((d0 + dd) * Np + n) * 4, 0, 0));
      }
    }
    __syncthreads();
    if (active) {
#pragma unroll
      for (int dd = 0; dd < DC; ++dd) {
        float kv[NK];
#pragma unroll
        for (int i = 0; i < NK; ++i) kv[i] = ksh[dd][lane + 64 * i];
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
          const float qv = __builtin_bit_cast(
              float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, qlane[rr]), d0 + dd));
#pragma unroll
          for (int i = 0; i < NK; ++i) acc[rr][i] = acc[rr][i] + qv * kv[i];
        }
      }
    }
  }
  if (!active) return;  // whole wave; no workgroup barrier below

#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    const int m = m0 + rr;
    if (m >= Mb) break;  // uniform
    uint32_t ord[NK];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int n = lane + 64 * i;
      ord[i] = n < Np ? (uint32_t)(score_key(acc[rr][i] * scale, n) >> 32) : 0u;  // 0: below all
    }
    // wave-wide sum of per-lane counts 0..NK: one ballot per count bit
    constexpr int kBits = NK == 8 ? 4 : (NK == 16 ? 5 : (NK == 32 ? 6 : 7));
    auto wave_sum = [&](int cl) {
      int c = 0;
#pragma unroll
      for (int b = 0; b < kBits; ++b) c += __popcll(__ballot((cl >> b) & 1)) << b;
      return c;
    };
    auto count_ge = [&](uint32_t v) {
      int cl = 0;
#pragma unroll
      for (int i = 0; i < NK; ++i) cl += ord[i] >= v ? 1 : 0;
      return wave_sum(cl);
    };
    uint32_t sstar = 0;
    for (int b = 31; b >= 0; --b) {
      const uint32_t cand = sstar | (1u << b);
      if (count_ge(cand) >= T) sstar = cand;
    }
    int l_gt = 0, l_eq = 0;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      l_gt += ord[i] > sstar ? 1 : 0;
      l_eq += ord[i] == sstar ? 1 : 0;
    }
    const int c_gt = wave_sum(l_gt), c_eq = wave_sum(l_eq);
    const int need = T - c_gt;  // 1 <= need <= c_eq
    uint32_t nstar = 0xffffffffu;  // tie keys with n <= nstar are taken
    if (need < c_eq) {
      uint32_t pre = 0;
      for (int b = 12; b >= 0; --b) {
        const uint32_t cand = pre | (1u << b);
        int cl = 0;
#pragma unroll
        for (int i = 0; i < NK; ++i) cl += (ord[i] == sstar && (uint32_t)(lane + 64 * i) < cand) ? 1 : 0;
        if (wave_sum(cl) < need) pre = cand;
      }
      nstar = pre;
    }
    // compact the T winners (any order), then sort them across the lanes
    int base = 0;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const uint32_t n = lane + 64 * i;
      const bool sel = ord[i] > sstar || (ord[i] == sstar && n <= nstar);
      const uint64_t bal = __ballot(sel);
      if (sel) {
        const int pos = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        win[w][pos] = ((uint64_t)ord[i] << 32) | (uint64_t)(0xffffffffu - n);
      }
      if (mask != nullptr && (int)n < Np) mask[((int64_t)bh * Mb + m) * Np + n] = sel ? 1 : 0;
      base += __popcll(bal);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    uint64_t key = lane < T ? win[w][lane] : 0ull;
    // bitonic sort, descending, over the 64 lanes
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
      for (int j = k >> 1; j > 0; j >>= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)key, j, 64);
        const uint32_t hi = __shfl_xor((uint32_t)(key >> 32), j, 64);
        const uint64_t other = ((uint64_t)hi << 32) | lo;
        const bool desc = (lane & k) == 0;
        const bool lower = (lane & j) == 0;  // this lane keeps the larger key in a desc run
        const bool take = desc == lower ? other > key : other < key;
        key = take ? other : key;
      }
    }
    if (lane < T) lut[((int64_t)bh * Mb + m) * T + lane] = (int32_t)(0xffffffffu - (uint32_t)key);
    __builtin_amdgcn_wave_barrier();  // win[w] is reused by the next row
  }
}

}  // namespace sla2h

using namespace sla2h;

// Workgroups cycling over tiles: 16 per CU of 256 (two rounds of eight
// resident ones; measured best among 1024-8192 at Config 3).
constexpr int kQuantGrid = 4096;

static int launch_quant_pool(const QuantPoolArgs& a, int ntens, int dtype, hipStream_t st) {
  const int64_t ntiles = (int64_t)a.Nb * ntens * a.BH;
  if (ntiles >= (1ll << 31) - (kQuantSets + 2) * (int64_t)kQuantGrid) return (int)hipErrorInvalidValue;
  const int grid = (int)(ntiles < kQuantGrid ? ntiles : kQuantGrid);
  if (dtype == SLA2H_DTYPE_BF16)
    quant_pool_kernel<BF16><<<grid, 256, 0, st>>>(a, (int)ntiles);
  else
    quant_pool_kernel<F16><<<grid, 256, 0, st>>>(a, (int)ntiles);
  return (int)hipGetLastError();
}

// Block means for the 1-D router (blocks of blk rows, the last one ragged):
// one block of one (b, h) per workgroup, one thread per channel, sequential
// fp32 sum over the block's real rows, then / count, then the optional
// projection out[e] = sum_d mean[d] proj[e][d] (sequential, no contraction).
// fp32 input "storage tag" for the pooling kernel (16-bit tags: common.h)
struct F32In {
  __device__ static inline float to_f32(float f) { return f; }
};

template <typename TS, typename Raw>
__global__ __launch_bounds__(64) void pool_blocks_kernel(const Raw* __restrict__ x, int64_t L,
                                                        int blk, int nblk,
                                                        const float* __restrict__ proj,
                                                        int transposed, float* __restrict__ out) {
  using T16 = TS;
  __shared__ float vec[kTile];
  const int j = blockIdx.x, bh = blockIdx.y, d = threadIdx.x;
  const int64_t r0 = (int64_t)j * blk;
  const int cnt = (int)((L - r0) < blk ? (L - r0) : blk);
  const Raw* src = x + ((int64_t)bh * L + r0) * kTile + d;
  float acc = 0.f;
  int rr = 0;
  for (; rr + 16 <= cnt; rr += 16) {  // 16 loads in flight, then the adds in row order
    float xv[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) xv[u] = T16::to_f32(src[(int64_t)(rr + u) * kTile]);
#pragma unroll
    for (int u = 0; u < 16; ++u) acc = acc + xv[u];
  }
  for (; rr < cnt; ++rr) acc = acc + T16::to_f32(src[(int64_t)rr * kTile]);
  vec[d] = acc / (float)cnt;
  __syncthreads();
  float outv = vec[d];
  if (proj != nullptr) {
    const float* pr = proj + d * kTile;
    float p = 0.f;
    for (int e = 0; e < kTile; ++e) p = p + vec[e] * pr[e];
    outv = p;
  }
  if (transposed)
    out[((int64_t)bh * kTile + d) * nblk + j] = outv;
  else
    out[((int64_t)bh * nblk + j) * kTile + d] = outv;
}

extern "C" int sla2h_pool_blocks(const void* x, int dtype, int64_t BH, int64_t L, int D, int blk,
                                 const float* proj, int transposed, float* out, void* stream) {
  SLA2H_CHECK_ARG(x && out);
  SLA2H_CHECK_ARG(D == kTile && blk >= 1 && blk <= 4096);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16 || dtype == 2);
  SLA2H_CHECK_ARG(BH > 0 && BH <= 65535 && L > 0);
  const int64_t nblk = (L + blk - 1) / blk;
  SLA2H_CHECK_ARG(nblk < (1ll << 31));
  dim3 grid((unsigned)nblk, (unsigned)BH);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto X = static_cast<const uint16_t*>(x);
  if (dtype == 2)
    pool_blocks_kernel<F32In, float><<<grid, kTile, 0, st>>>(static_cast<const float*>(x), L, blk,
                                                            (int)nblk, proj, transposed, out);
  else if (dtype == SLA2H_DTYPE_BF16)
    pool_blocks_kernel<BF16, uint16_t><<<grid, kTile, 0, st>>>(X, L, blk, (int)nblk, proj,
                                                              transposed, out);
  else
    pool_blocks_kernel<F16, uint16_t><<<grid, kTile, 0, st>>>(X, L, blk, (int)nblk, proj,
                                                             transposed, out);
  return (int)hipGetLastError();
}

extern "C" int sla2h_version(void) { return 1; }

extern "C" const char* sla2h_error_string(int code) {
  return hipGetErrorString((hipError_t)code);
}

extern "C" int sla2h_quant_train(const void* q, const void* k, const void* v, int dtype, int B,
                                 int H, int64_t L, int D, int E, int8_t* q8, float* qs, int8_t* k8,
                                 float* ks, int8_t* v8f, float* vs, void* stream) {
  SLA2H_CHECK_ARG(q && k && v && q8 && qs && k8 && ks && v8f && vs);
  SLA2H_CHECK_ARG(D == kTile && E == kTile);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && 3 * B * H <= 65535 && L > 0);
  QuantTrainArgs a;
  a.x[0] = static_cast<const uint16_t*>(q);
  a.x[1] = static_cast<const uint16_t*>(k);
  a.x[2] = static_cast<const uint16_t*>(v);
  a.xq[0] = q8;
  a.xq[1] = k8;
  a.xq[2] = v8f;
  a.xs[0] = qs;
  a.xs[1] = ks;
  a.xs[2] = vs;
  a.BH = B * H;
  a.L = L;
  a.Nb = (int)((L + E - 1) / E);
  a.t0 = 0;
  dim3 grid(a.Nb, 3 * a.BH);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SLA2H_DTYPE_BF16)
    quant_train_kernel<BF16><<<grid, 256, 0, st>>>(a);
  else
    quant_train_kernel<F16><<<grid, 256, 0, st>>>(a);
  return (int)hipGetLastError();
}

// The training kernel's truncating law (sla2h_quant_train) for one tensor in
// blocks of E = 32..256 rows: Q of the 1-D SLA2 INT8 training forward, whose
// query tiles are bq rows.
extern "C" int sla2h_quantize_trunc(const void* x, int dtype, int64_t BH, int64_t L, int D,
                                    int E, int8_t* xq, float* xs, void* stream) {
  SLA2H_CHECK_ARG(x && xq && xs);
  SLA2H_CHECK_ARG(D == kTile && (E == 32 || E == 64 || E == 128 || E == 256));
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(BH > 0 && BH <= 65535 && L > 0);
  const int Nb = (int)((L + E - 1) / E);
  dim3 grid(Nb, (int)BH);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto X = static_cast<const uint16_t*>(x);
  auto go = [&](auto tag) {
    using T16 = decltype(tag);
    if (E == 32)
      quant_rows_kernel<T16, 32, true><<<grid, 256, 0, st>>>(X, L, Nb, xq, xs);
    else if (E == 64)
      quant_rows_kernel<T16, 64, true><<<grid, 256, 0, st>>>(X, L, Nb, xq, xs);
    else if (E == 128)
      quant_rows_kernel<T16, 128, true><<<grid, 256, 0, st>>>(X, L, Nb, xq, xs);
    else
      quant_rows_kernel<T16, 256, true><<<grid, 256, 0, st>>>(X, L, Nb, xq, xs);
  };
  if (dtype == SLA2H_DTYPE_BF16)
    go(BF16{});
  else
    go(F16{});
  return (int)hipGetLastError();
}

// V of the inference INT8 path: quantize_qkv's law (round half away, one
// scale per 64-row block) written in the INT8 MFMA fragment order of the
// sparse kernels (the layout of sla2h_quant_train's v8f).
extern "C" int sla2h_quantize_v8f(const void* v, int dtype, int64_t BH, int64_t L, int D, int E,
                                  int8_t* v8f, float* vs, void* stream) {
  SLA2H_CHECK_ARG(v && v8f && vs);
  SLA2H_CHECK_ARG(D == kTile && E == kTile);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(BH > 0 && BH <= 65535 && L > 0);
  QuantTrainArgs a = {};
  a.x[2] = static_cast<const uint16_t*>(v);
  a.xq[2] = v8f;
  a.xs[2] = vs;
  a.BH = (int)BH;
  a.L = L;
  a.Nb = (int)((L + E - 1) / E);
  a.t0 = 2;
  dim3 grid(a.Nb, (int)BH);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SLA2H_DTYPE_BF16)
    quant_train_kernel<BF16, true><<<grid, 256, 0, st>>>(a);
  else
    quant_train_kernel<F16, true><<<grid, 256, 0, st>>>(a);
  return (int)hipGetLastError();
}

extern "C" int sla2h_quantize(const void* x, int dtype, int64_t BH, int64_t L, int D, int E,
                              int8_t* xq, float* xs, void* stream) {
  SLA2H_CHECK_ARG(x && xq && xs);
  SLA2H_CHECK_ARG(D == kTile && (E == 32 || E == 64 || E == 128 || E == 256));
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(BH > 0 && BH <= 65535 && L > 0);
  if (BH * L * D == 0) return 0;
  if (E != kTile) {
    const int Nb = (int)((L + E - 1) / E);
    dim3 grid(Nb, (int)BH);
    hipStream_t st = static_cast<hipStream_t>(stream);
    auto X = static_cast<const uint16_t*>(x);
    auto go = [&](auto tag) {
      using T16 = decltype(tag);
      if (E == 32)
        quant_rows_kernel<T16, 32><<<grid, 256, 0, st>>>(X, L, Nb, xq, xs);
      else if (E == 128)
        quant_rows_kernel<T16, 128><<<grid, 256, 0, st>>>(X, L, Nb, xq, xs);
      else
        quant_rows_kernel<T16, 256><<<grid, 256, 0, st>>>(X, L, Nb, xq, xs);
    };
    if (dtype == SLA2H_DTYPE_BF16)
      go(BF16{});
    else
      go(F16{});
    return (int)hipGetLastError();
  }
  QuantPoolArgs a = {};
  a.x[0] = static_cast<const uint16_t*>(x);
  a.xq[0] = xq;
  a.xs[0] = xs;
  a.BH = (int)BH;
  a.L = L;
  a.Nb = (int)((L + E - 1) / E);
  return launch_quant_pool(a, 1, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int sla2h_quant_pool_qk(const void* q, const void* k, int dtype, int B, int H,
                                   int64_t L, int D, int E, int Np, const float* proj_q,
                                   const float* proj_k, int8_t* q8, float* qs, int8_t* k8,
                                   float* ks, float* qpool, float* kpool_t, float* kbound,
                                   void* stream) {
  SLA2H_CHECK_ARG(q && k && q8 && qs && k8 && ks && qpool && kpool_t);
  SLA2H_CHECK_ARG(D == kTile && E == kTile);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && (int64_t)B * H * 2 <= 65535);
  SLA2H_CHECK_ARG(Np > 0 && (int64_t)Np * E <= L);
  QuantPoolArgs a = {};
  a.BH = B * H;
  a.L = L;
  a.Nb = (int)((L + E - 1) / E);
  a.x[0] = static_cast<const uint16_t*>(q);
  a.x[1] = static_cast<const uint16_t*>(k);
  a.xq[0] = q8;
  a.xq[1] = k8;
  a.xs[0] = qs;
  a.xs[1] = ks;
  a.pool[0] = qpool;
  a.pool[1] = kpool_t;
  a.proj[0] = proj_q;
  a.proj[1] = proj_k;
  a.npool[0] = a.Nb;
  a.npool[1] = Np;
  a.pool_len[0] = L;
  a.pool_len[1] = (int64_t)Np * E;
  a.transposed[0] = 0;
  a.transposed[1] = 1;
  a.kb[1] = kbound;
  return launch_quant_pool(a, 2, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int sla2h_route_topk(const float* qpool, const float* kpool_t, int B, int H, int Mb,
                                int Np, int D, int T, float scale, int32_t* lut, uint8_t* mask,
                                void* stream) {
  SLA2H_CHECK_ARG(qpool && kpool_t && lut);
  SLA2H_CHECK_ARG(D == kTile);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && B * H <= 65535 && Mb > 0);
  SLA2H_CHECK_ARG(Np > 0 && Np <= 4096 && T >= 1 && T <= Np);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (T <= 64) {
    // one query block per wave: enough waves to hide the load latency
    auto go = [&](auto nk, auto rows) {
      constexpr int NK = decltype(nk)::value, R = decltype(rows)::value;
      dim3 grid((Mb + 4 * R - 1) / (4 * R), B * H);
      if (Np % 4 == 0)
        route_select_kernel<NK, R, true><<<grid, 256, 0, st>>>(qpool, kpool_t, Mb, Np, T, scale, lut, mask);
      else
        route_select_kernel<NK, R, false><<<grid, 256, 0, st>>>(qpool, kpool_t, Mb, Np, T, scale, lut, mask);
    };
    if (Np <= 512)
      go(std::integral_constant<int, 8>{}, std::integral_constant<int, 1>{});
    else if (Np <= 1024)
      go(std::integral_constant<int, 16>{}, std::integral_constant<int, 1>{});
    else if (Np <= 2048)
      go(std::integral_constant<int, 32>{}, std::integral_constant<int, 1>{});
    else
      go(std::integral_constant<int, 64>{}, std::integral_constant<int, 1>{});
    return (int)hipGetLastError();
  }
  int P2 = 1;
  while (P2 < Np) P2 <<= 1;
  if (P2 < 2) P2 = 2;
  const int rows = P2 <= 512 ? 8 : (P2 <= 1024 ? 4 : (P2 <= 2048 ? 2 : 1));
  const size_t shmem = (size_t)rows * P2 * 8 + (size_t)rows * kTile * 4 + (size_t)rows * P2;
  dim3 grid((Mb + rows - 1) / rows, B * H);
  switch (rows) {
    case 8: route_topk_kernel<8><<<grid, 256, shmem, st>>>(qpool, kpool_t, Mb, Np, T, scale, P2, lut, mask); break;
    case 4: route_topk_kernel<4><<<grid, 256, shmem, st>>>(qpool, kpool_t, Mb, Np, T, scale, P2, lut, mask); break;
    case 2: route_topk_kernel<2><<<grid, 256, shmem, st>>>(qpool, kpool_t, Mb, Np, T, scale, P2, lut, mask); break;
    default: route_topk_kernel<1><<<grid, 256, shmem, st>>>(qpool, kpool_t, Mb, Np, T, scale, P2, lut, mask); break;
  }
  return (int)hipGetLastError();
}
