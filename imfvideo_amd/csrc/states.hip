// Linear-branch states (phi(K)^T V per video tile, their tangents and global
// sums), the transposed value tiles used by the attention kernel, and the
// per-query-block complement records.
//
// Reference semantics:
//   phi / states   models/sla2_cube_qat.py:911-958 (_phi_states_kernel)
//   global sums    models/sla2_cube_qat.py:645-648
//   complement     models/sla2_cube_qat.py:510-523, 570-578
#include "common.h"

#include <mutex>

namespace sla2h {

constexpr int kT = 64;          // E = D = 64
constexpr int kLds = kT + 8;    // padded LDS row (16-bit elements)
constexpr size_t kRecBytes = 2 * 16384 + 2 * 256;

// One tile (b,h,n) per workgroup.  n < Np: phi, states; every n < Nb: the
// attention kernel's operand tiles, in MFMA fragment order so that each wave
// load there is one contiguous 1 KB (rows past L are zero).  With lane
// (g, r) = (lane/16, lane%16), wave w = keys 16w..16w+15, column tile ct:
//   vt, tangent: [ct][w][lane] 16 B = V[16w+4g+0..3][16ct+r] | dV[same]
//   vt, primal:  [ct][w][lane]  8 B = V[16w+4g+0..3][16ct+r]
//   kt (tangent only): [w][ks][lane] 16 B = K[16w+r][32ks+8g+0..7] for ks 0,1,
//                      dK[16w+r][32(ks-2)+8g+0..7] for ks 2,3
//
// Products phi^T V run on 16-bit MFMA with phi split into hi + lo halves of
// the input's 16-bit type (about 16 significant bits), fp32 accumulate.
// ROUND (training forward): phi is rounded to the 16-bit type first, as the
// reference's softmax(K).to(dtype) (models/sla2_cube_qat.py:728), and the lo
// half vanishes.  RH (the inference states of _hblocks): H is stored
// rounded to the 16-bit type, as the reference keeps HALL in V's dtype.  The
// value operand tiles are written when vt is not NULL.
template <typename T16, bool TAN, bool ROUND = false, bool RH = false>
__global__ __launch_bounds__(256) void linear_states_kernel(
    const uint16_t* __restrict__ K, const uint16_t* __restrict__ dK,
    const uint16_t* __restrict__ V, const uint16_t* __restrict__ dV, int64_t L, int Np, int Nb,
    float* __restrict__ Hb, float* __restrict__ dHb, float* __restrict__ zb,
    float* __restrict__ dzb, uint16_t* __restrict__ vt, uint16_t* __restrict__ kt) {
  // phi^T, then (tangent, second phase) dphi^T: one buffer keeps the LDS
  // footprint at four workgroups per CU
  __shared__ __align__(16) uint16_t phiT[2][kT][kLds];   // [hi/lo][d][r]
  __shared__ __align__(16) uint16_t vT[kT][kLds];        // [c][r]
  __shared__ __align__(16) uint16_t dvT[kT][kLds];
  __shared__ float zred[2][4][kT];

  const int tid = threadIdx.x;
  const int n = blockIdx.x;
  const int bh = blockIdx.y;
  const int r = tid >> 2;
  const int c0 = (tid & 3) * 16;
  const int64_t row = (int64_t)n * kT + r;
  const bool valid = row < L;
  const int64_t off = ((int64_t)bh * L + row) * kT + c0;

  auto load16 = [&](const uint16_t* src, uint16_t* dst) {
    if (valid) {
      const uint4* s = reinterpret_cast<const uint4*>(src + off);
      uint4 u0 = s[0], u1 = s[1];
      uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        dst[2 * i] = (uint16_t)(w[i] & 0xffff);
        dst[2 * i + 1] = (uint16_t)(w[i] >> 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) dst[i] = 0;
    }
  };

  uint16_t vb[16], dvb[16];
  load16(V, vb);
  if (TAN) load16(dV, dvb);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    vT[c0 + i][r] = vb[i];
    if (TAN) dvT[c0 + i][r] = dvb[i];
  }

  const bool states = n < Np;  // uniform over the workgroup
  uint16_t kb[16], dkb[16];
  if (states || TAN) {
    load16(K, kb);
    if (TAN) load16(dK, dkb);
  }
  if (TAN) {  // key-operand fragments of this thread's 16 columns: 2 x (K, dK) chunks
    const int kw = r >> 4, rr = r & 15, ksd = c0 >> 5, g0 = (c0 & 31) >> 3;
    unsigned char* base = reinterpret_cast<unsigned char*>(kt) + ((int64_t)bh * Nb + n) * 16384;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int lane = (g0 + h2) * 16 + rr;
      uint4 kv, dkv;
      kv.x = pack2(kb[8 * h2 + 0], kb[8 * h2 + 1]); kv.y = pack2(kb[8 * h2 + 2], kb[8 * h2 + 3]);
      kv.z = pack2(kb[8 * h2 + 4], kb[8 * h2 + 5]); kv.w = pack2(kb[8 * h2 + 6], kb[8 * h2 + 7]);
      dkv.x = pack2(dkb[8 * h2 + 0], dkb[8 * h2 + 1]); dkv.y = pack2(dkb[8 * h2 + 2], dkb[8 * h2 + 3]);
      dkv.z = pack2(dkb[8 * h2 + 4], dkb[8 * h2 + 5]); dkv.w = pack2(dkb[8 * h2 + 6], dkb[8 * h2 + 7]);
      *reinterpret_cast<uint4*>(base + ((kw * 4 + ksd) * 64 + lane) * 16) = kv;
      *reinterpret_cast<uint4*>(base + ((kw * 4 + ksd + 2) * 64 + lane) * 16) = dkv;
    }
  }
  float dphi[16];
  if (states) {
    float x[16], phi[16];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      x[i] = T16::to_f32(kb[i]);
      mx = fmaxf(mx, x[i]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    float den = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      phi[i] = __expf(x[i] - mx);
      den += phi[i];
    }
    den += __shfl_xor(den, 1, 64);
    den += __shfl_xor(den, 2, 64);
#pragma unroll
    for (int i = 0; i < 16; ++i) phi[i] = phi[i] / den;
    if (TAN) {
      float dot = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) dot += phi[i] * T16::to_f32(dkb[i]);
      dot += __shfl_xor(dot, 1, 64);
      dot += __shfl_xor(dot, 2, 64);
#pragma unroll
      for (int i = 0; i < 16; ++i) dphi[i] = phi[i] * (T16::to_f32(dkb[i]) - dot);
    }
    if (!valid) {  // padding rows of a ragged last tile stay inert
#pragma unroll
      for (int i = 0; i < 16; ++i) phi[i] = dphi[i] = 0.f;
    }
    if (ROUND) {
#pragma unroll
      for (int i = 0; i < 16; ++i) phi[i] = T16::to_f32(T16::from_f32(phi[i]));
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint16_t hi = T16::from_f32(phi[i]);
      phiT[0][c0 + i][r] = hi;
      phiT[1][c0 + i][r] = T16::from_f32(phi[i] - T16::to_f32(hi));
    }
    // column sums over the 64 rows: 16 rows per wave by shuffles, then LDS
    const int w = tid >> 6;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s = phi[i];
      float ds = TAN ? dphi[i] : 0.f;
#pragma unroll
      for (int m = 4; m <= 32; m <<= 1) {
        s += __shfl_xor(s, m, 64);
        if (TAN) ds += __shfl_xor(ds, m, 64);
      }
      if ((tid & 63) < 4) {
        zred[0][w][c0 + i] = s;
        if (TAN) zred[1][w][c0 + i] = ds;
      }
    }
  }
  __syncthreads();

  // value-operand tile in fragment order: thread -> (ct, w, r), 4 lane groups g
  if (vt != nullptr) {
    const int ct = tid >> 6, vw = (tid >> 4) & 3, rr = tid & 15;
    const int c = 16 * ct + rr;
    unsigned char* base = reinterpret_cast<unsigned char*>(vt) +
                          ((int64_t)bh * Nb + n) * (TAN ? 16384 : 8192);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int lane = g * 16 + rr;
      const int k0 = 16 * vw + 4 * g;
      const uint2 a = *reinterpret_cast<const uint2*>(&vT[c][k0]);
      if (TAN) {
        const uint2 b = *reinterpret_cast<const uint2*>(&dvT[c][k0]);
        *reinterpret_cast<uint4*>(base + ((ct * 4 + vw) * 64 + lane) * 16) = make_uint4(a.x, a.y, b.x, b.y);
      } else {
        *reinterpret_cast<uint2*>(base + ((ct * 4 + vw) * 64 + lane) * 8) = a;
      }
    }
  }
  if (!states) return;

  if (tid < kT) {
    const int64_t zo = ((int64_t)bh * Np + n) * kT + tid;
    zb[zo] = (zred[0][0][tid] + zred[0][1][tid]) + (zred[0][2][tid] + zred[0][3][tid]);
    if (TAN) dzb[zo] = (zred[1][0][tid] + zred[1][1][tid]) + (zred[1][2][tid] + zred[1][3][tid]);
  }

  // Hb[d][v] = sum_r phi[r][d] V[r][v]: wave w owns d rows 16w..16w+15.
  const int w = tid >> 6, l = tid & 63, lr = l & 15, g = l >> 4;
  const int drow = 16 * w + lr;
  f32x4 acc[4], dacc[4];
#pragma unroll
  for (int vt_ = 0; vt_ < 4; ++vt_) {
    acc[vt_] = f32x4{0.f, 0.f, 0.f, 0.f};
    dacc[vt_] = acc[vt_];
  }
  // phase 1: H = phi^T V and the phi^T dV half of dH
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int k0 = 32 * ks + 8 * g;
    const u32x4 ah = *reinterpret_cast<const u32x4*>(&phiT[0][drow][k0]);
    const u32x4 al = *reinterpret_cast<const u32x4*>(&phiT[1][drow][k0]);
#pragma unroll
    for (int vt_ = 0; vt_ < 4; ++vt_) {
      const u32x4 bv = *reinterpret_cast<const u32x4*>(&vT[16 * vt_ + lr][k0]);
      acc[vt_] = mfma_16x16x32<T16>(ah, bv, acc[vt_]);
      if (!ROUND) acc[vt_] = mfma_16x16x32<T16>(al, bv, acc[vt_]);
      if (TAN) {
        const u32x4 bdv = *reinterpret_cast<const u32x4*>(&dvT[16 * vt_ + lr][k0]);
        dacc[vt_] = mfma_16x16x32<T16>(ah, bdv, dacc[vt_]);
        dacc[vt_] = mfma_16x16x32<T16>(al, bdv, dacc[vt_]);
      }
    }
  }
  if (TAN) {  // phase 2: dphi^T replaces phi^T; dH += dphi^T V
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint16_t dhi = T16::from_f32(dphi[i]);
      phiT[0][c0 + i][r] = dhi;
      phiT[1][c0 + i][r] = T16::from_f32(dphi[i] - T16::to_f32(dhi));
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int k0 = 32 * ks + 8 * g;
      const u32x4 dah = *reinterpret_cast<const u32x4*>(&phiT[0][drow][k0]);
      const u32x4 dal = *reinterpret_cast<const u32x4*>(&phiT[1][drow][k0]);
#pragma unroll
      for (int vt_ = 0; vt_ < 4; ++vt_) {
        const u32x4 bv = *reinterpret_cast<const u32x4*>(&vT[16 * vt_ + lr][k0]);
        dacc[vt_] = mfma_16x16x32<T16>(dah, bv, dacc[vt_]);
        dacc[vt_] = mfma_16x16x32<T16>(dal, bv, dacc[vt_]);
      }
    }
  }
  const int64_t hbase = ((int64_t)bh * Np + n) * kT * kT;
#pragma unroll
  for (int vt_ = 0; vt_ < 4; ++vt_) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t o = hbase + (int64_t)(16 * w + 4 * g + i) * kT + 16 * vt_ + lr;
      Hb[o] = RH ? T16::to_f32(T16::from_f32(acc[vt_][i])) : acc[vt_][i];
      if (TAN) dHb[o] = dacc[vt_][i];
    }
  }
}

// Global sums over the Np tiles in a fixed order (deterministic): four
// contiguous ranges of tiles summed in sequence by four threads of a column,
// then ((r0 + r1) + (r2 + r3)).  64 columns per workgroup of 256 threads.
// Column index e spans [Hb 4096 | dHb 4096 | zb 64 | dzb 64].
__global__ __launch_bounds__(256) void states_sum_kernel(const float* __restrict__ Hb,
                                                        const float* __restrict__ dHb,
                                                        const float* __restrict__ zb,
                                                        const float* __restrict__ dzb, int Np,
                                                        float* __restrict__ Hall,
                                                        float* __restrict__ dHall,
                                                        float* __restrict__ zall,
                                                        float* __restrict__ dzall) {
  __shared__ float part[4][64];
  const int c = threadIdx.x & 63, part_id = threadIdx.x >> 6;
  const int e = blockIdx.x * 64 + c;
  const int bh = blockIdx.y;
  const float* src;
  float* dst;
  int stride, col;
  if (e < 4096) {
    src = Hb; dst = Hall; stride = 4096; col = e;
  } else if (e < 8192) {
    src = dHb; dst = dHall; stride = 4096; col = e - 4096;
  } else if (e < 8256) {
    src = zb; dst = zall; stride = 64; col = e - 8192;
  } else {
    src = dzb; dst = dzall; stride = 64; col = e - 8256;
  }
  if (src == nullptr) return;  // uniform: a workgroup never spans two parts
  const int chunk = (Np + 3) / 4;
  const int n0 = part_id * chunk, n1 = min(Np, n0 + chunk);
  const float* p = src + (int64_t)bh * Np * stride + col;
  float acc = 0.f;
#pragma unroll 8
  for (int nn = n0; nn < n1; ++nn) acc += p[(int64_t)nn * stride];
  part[part_id][c] = acc;
  __syncthreads();
  if (part_id == 0)
    dst[(int64_t)bh * stride + col] = (part[0][c] + part[1][c]) + (part[2][c] + part[3][c]);
}

// ---------------------------------------------------------------------------
// Complement records.  For each query block m of a head:
//   Hc[m] = sum over the video tiles n NOT routed for m of Hb[n]   (and dHc, zc, dzc)
// computed as a GEMM per head, C = Mc . S, with Mc[m][n] = 1 - sel(m, n)
// (Mb x Np, 0/1) and S = [Hb | dHb | zb | dzb] (Np x 8320 columns, fp32).  S
// is split into bf16 hi + lo halves (about 16 significant bits) and the
// products accumulate in fp32 on MFMA; the mask is exact in bf16.  The H
// columns run in comp_gemm_kernel, the z columns in comp_mask_kernel.
//
// Record of (b,h,m), kRecBytes bytes, fp32:
//   [0, 16384) Hc[d][v] row-major, [16384, 32768) dHc, [32768, 33024) zc,
//   [33024, 33280) dzc.
// ---------------------------------------------------------------------------
constexpr int kMaskSub = 32;  // 16-row mask sub-tiles per GEMM workgroup (512 rows)
constexpr int kCompCols = 64;  // state columns per GEMM workgroup
constexpr int kCompThreads = 512;  // 8 waves

// 8 mask bits -> the 8 bf16 A-operand slots (1.0 where set)
__device__ __forceinline__ u32x4 expand_mask8(uint32_t b) {
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t v = (b >> (2 * e)) & 3u;
    o[e] = ((v & 1u) | ((v & 2u) << 15)) * 0x3F80u;
  }
  return o;
}

// Complement bit masks cbits[bh][kc][m] (m < 16 MT): bit j of word (kc, m) is
// 1 where tile n = 32 kc + j < Np is not routed for query block m < Mb.
// With zb given, the workgroup also writes the zc (and, with dzb, dzc) parts
// of its 16 query blocks' records: the same 0/1-mask product as the GEMM
// below (bf16 hi + lo halves of zb, chunks of 32 tiles in the same order).
// Wave w owns columns 16 (w % 4) .. + 15 of zc (w < 4) or of dzc (w >= 4,
// eight waves with the tangent).  This keeps the 64- and 128-column z parts
// out of the GEMM's grid.
__global__ __launch_bounds__(512) void comp_mask_kernel(const int32_t* __restrict__ lut, int Mb,
                                                      int Np, int T, int MT, int NC,
                                                      uint32_t* __restrict__ cbits,
                                                      const float* __restrict__ zb,
                                                      const float* __restrict__ dzb,
                                                      unsigned char* __restrict__ comp) {
  extern __shared__ uint32_t selbits[];  // [16][NC]
  const int mt = blockIdx.x, bh = blockIdx.y, tid = threadIdx.x;
  const int nthr = blockDim.x;
  for (int i = tid; i < 16 * NC; i += nthr) selbits[i] = 0u;
  __syncthreads();
  for (int i = tid; i < 16 * T; i += nthr) {
    const int row = i / T, jj = i % T;
    const int m = mt * 16 + row;
    if (m >= Mb) continue;
    const int n = lut[((int64_t)bh * Mb + m) * T + jj];
    if ((unsigned)n < (unsigned)Np) atomicOr(&selbits[row * NC + (n >> 5)], 1u << (n & 31));
  }
  __syncthreads();
  for (int i = tid; i < NC * 16; i += nthr) {
    const int kc = i >> 4, row = i & 15;
    const int m = mt * 16 + row;
    const int nv = Np - 32 * kc;  // real tiles in this word
    const uint32_t valid = nv >= 32 ? 0xffffffffu : ((1u << nv) - 1u);
    cbits[((int64_t)bh * NC + kc) * (MT * 16) + m] = m < Mb ? (~selbits[row * NC + kc] & valid) : 0u;
  }
  if (zb == nullptr) return;

  const int w = tid >> 6, l = tid & 63, r = l & 15, g = l >> 4;
  const int part = w >> 2, cw = w & 3;  // part 0: zc from zb, 1: dzc from dzb
  const bool rowok = mt * 16 + r < Mb;
  // tiles n >= Np read as 0 (buffer range check); four chunks of loads in flight
  const auto rz = make_rsrc((part ? dzb : zb) + (int64_t)bh * Np * kT, (int64_t)Np * kT * 4);
  const int coff = (16 * cw + r) * 4;
  auto split = [](const float* x, u32x4& hi, u32x4& lo) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t h = pack_pair<BF16>(x[2 * e], x[2 * e + 1]);
      hi[e] = h;
      lo[e] = pack_pair<BF16>(x[2 * e] - __builtin_bit_cast(float, h << 16),
                              x[2 * e + 1] - __builtin_bit_cast(float, h & 0xffff0000u));
    }
  };
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  constexpr int kU = 4;
  for (int kc0 = 0; kc0 < NC; kc0 += kU) {
    float x[kU][8];
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int off = (32 * (kc0 + u) + 8 * g + j) * (kT * 4) + coff;
        x[u][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rz, off, 0, 0));
      }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int kc = kc0 + u;
      if (kc >= NC) break;
      const int nv = Np - 32 * kc;
      const uint32_t valid = nv >= 32 ? 0xffffffffu : ((1u << nv) - 1u);
      const uint32_t word = rowok ? (~selbits[r * NC + kc] & valid) : 0u;
      const u32x4 am = expand_mask8((word >> (8 * g)) & 0xffu);
      u32x4 hi, lo;
      split(x[u], hi, lo);
      acc = mfma_bf16_16x16x32(am, hi, acc);
      acc = mfma_bf16_16x16x32(am, lo, acc);
    }
  }
  // lane (g, r) element i = C[query block 16 mt + 4g + i][column 16 cw + r]
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = mt * 16 + 4 * g + i;
    if (m >= Mb) continue;
    unsigned char* rec = comp + ((int64_t)bh * Mb + m) * kRecBytes;
    reinterpret_cast<float*>(rec + 32768 + 256 * part)[16 * cw + r] = acc[i];
  }
}

// One workgroup of 8 waves: 64 state columns x up to 512 query blocks of one
// head (wave w owns the 16-row tiles w, w+8, w+16, w+24, so 64 accumulator
// registers per lane and four waves per SIMD).  The contraction over video
// tiles runs in chunks of 32, double-buffered in LDS and prefetched two
// chunks ahead.  Staging: thread (wave w, column c) loads rows 4w..4w+3 of
// column c, splits them into bf16 hi + lo and writes half a B-operand
// fragment of each with one 8-byte LDS store.  The A operand (0/1 mask)
// comes from the row's mask byte, one 16-entry nibble table read per half.
template <bool TAN>
__global__ __launch_bounds__(kCompThreads, 4) void comp_gemm_kernel(
    const float* __restrict__ Hb, const float* __restrict__ dHb, const float* __restrict__ zb,
    const float* __restrict__ dzb, const uint32_t* __restrict__ cbits, int Mb, int Np, int MT,
    int NC, unsigned char* __restrict__ comp) {
  __shared__ __align__(16) uint16_t sb[2][2][kCompCols][40];  // [buf][hi/lo][column][n] (+pad)
  __shared__ __align__(16) uint32_t mw[2][16 * kMaskSub];    // [buf][local row] mask words
  // mask nibble -> four bf16 operand slots: 16 entries of 8 bytes occupy 32 distinct LDS
  // banks, so lanes reading different entries never conflict
  __shared__ __align__(16) u32x2 mexp[16];

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, r = l & 15, g = l >> 4;
  const int c0 = blockIdx.x * kCompCols;
  const int bh = blockIdx.y;
  const int mt0 = blockIdx.z * kMaskSub;
  const int MTp = MT * 16;
  const int m0 = mt0 * 16;

  // column tile -> source tensor (boundaries are multiples of 64)
  const float* src;
  int stride, col0, part;  // part: 0 Hc, 1 dHc, 2 zc, 3 dzc
  const int zbase = TAN ? 8192 : 4096;
  if (c0 < 4096) {
    src = Hb; stride = 4096; col0 = c0; part = 0;
  } else if (TAN && c0 < 8192) {
    src = dHb; stride = 4096; col0 = c0 - 4096; part = 1;
  } else if (c0 < zbase + 64) {
    src = zb; stride = 64; col0 = c0 - zbase; part = 2;
  } else {
    src = dzb; stride = 64; col0 = c0 - zbase - 64; part = 3;
  }
  // tile rows n >= Np and mask words past the head read as 0 (buffer range check)
  const auto rs = make_rsrc(src + (int64_t)bh * Np * stride, (int64_t)Np * stride * 4);
  const auto rb = make_rsrc(cbits + (int64_t)bh * NC * MTp, (int64_t)NC * MTp * 4);

  if (tid < 16) {
    const u32x4 e = expand_mask8(tid);
    mexp[tid] = u32x2{e[0], e[1]};
  }

  f32x4 acc[4][4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[s][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

  struct Chunk {
    float x[4];
    uint32_t mk;
  };
  const int xoff = (col0 + l) * 4 + 4 * w * stride * 4;
  auto load_chunk = [&](int kc, Chunk& c) {
    kc = min(kc, NC - 1);  // past the end: a harmless reload, never stored
#pragma unroll
    for (int j = 0; j < 4; ++j)
      c.x[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             rs, xoff + (32 * kc + j) * stride * 4, 0, 0));
    c.mk = __builtin_amdgcn_raw_buffer_load_b32(rb, (kc * MTp + m0 + tid) * 4, 0, 0);
  };
  auto store_chunk = [&](int buf, const Chunk& c) {
    u32x2 hi, lo;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t h = pack_pair<BF16>(c.x[2 * e], c.x[2 * e + 1]);
      hi[e] = h;
      lo[e] = pack_pair<BF16>(c.x[2 * e] - __builtin_bit_cast(float, h << 16),
                              c.x[2 * e + 1] - __builtin_bit_cast(float, h & 0xffff0000u));
    }
    *reinterpret_cast<u32x2*>(&sb[buf][0][l][4 * w]) = hi;
    *reinterpret_cast<u32x2*>(&sb[buf][1][l][4 * w]) = lo;
    mw[buf][tid] = c.mk;
  };
  const unsigned char* mwb = reinterpret_cast<const unsigned char*>(&mw[0][0]);
  auto compute = [&](int buf) {
    u32x4 bhi[4], blo[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      bhi[ct] = *reinterpret_cast<const u32x4*>(&sb[buf][0][ct * 16 + r][8 * g]);
      blo[ct] = *reinterpret_cast<const u32x4*>(&sb[buf][1][ct * 16 + r][8 * g]);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int lt = w + 8 * s;  // local 16-row tile; uniform per wave
      if (mt0 + lt < MT) {
        const uint32_t mb = mwb[(buf * 16 * kMaskSub + lt * 16 + r) * 4 + g];
        const u32x2 alo = mexp[mb & 15u], ahi = mexp[mb >> 4];
        const u32x4 am = u32x4{alo.x, alo.y, ahi.x, ahi.y};
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          acc[s][ct] = mfma_bf16_16x16x32(am, bhi[ct], acc[s][ct]);
          acc[s][ct] = mfma_bf16_16x16x32(am, blo[ct], acc[s][ct]);
        }
      }
    }
  };

  Chunk ca, cb;
  load_chunk(0, ca);
  load_chunk(1, cb);
  store_chunk(0, ca);
  __syncthreads();
  for (int kc = 0; kc < NC; kc += 2) {
    // chunk kc in buffer 0, chunk kc+1 in registers cb
    load_chunk(kc + 2, ca);
    compute(0);
    store_chunk(1, cb);  // buffer 1 was last read before the previous barrier
    __syncthreads();
    if (kc + 1 >= NC) break;
    load_chunk(kc + 3, cb);
    compute(1);
    store_chunk(0, ca);
    __syncthreads();
  }

  // records: lane (g, r) element i = C[16 mt + 4g + i][c0 + 16 ct + r]; 16
  // consecutive columns of one record per 16 lanes
  const int pbase = part < 2 ? part * 16384 : 32768 + (part - 2) * 256;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int mt = mt0 + w + 8 * s;
    if (mt >= MT) break;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = mt * 16 + 4 * g + i;
      if (m >= Mb) continue;
      float* rec = reinterpret_cast<float*>(comp + ((int64_t)bh * Mb + m) * kRecBytes + pbase);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) rec[col0 + ct * 16 + r] = acc[s][ct][i];
    }
  }
}

}  // namespace sla2h

using namespace sla2h;

extern "C" size_t sla2h_complement_record_bytes(int D) { return D == kT ? kRecBytes : 0; }

extern "C" int sla2h_linear_states(const void* k, const void* dk, const void* v, const void* dv,
                                   int dtype, int B, int H, int64_t L, int D, int E, int Np,
                                   float* Hb, float* dHb, float* zb, float* dzb, float* Hall,
                                   float* dHall, float* zall, float* dzall, void* vt, void* kt,
                                   void* stream) {
  SLA2H_CHECK_ARG(k && v && Hb && zb && vt);
  SLA2H_CHECK_ARG((Hall == nullptr) == (zall == nullptr));
  SLA2H_CHECK_ARG(D == kT && E == kT);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && B * H <= 65535);
  // Np * E <= L for cube video tiles; Np = Nb (every tile, the last one
  // possibly partial) for 1-D key blocks
  SLA2H_CHECK_ARG(Np > 0 && (int64_t)(Np - 1) * E < L);
  const bool tan = dk != nullptr;
  if (tan) SLA2H_CHECK_ARG(dv && dHb && dzb && kt);
  if (tan && Hall) SLA2H_CHECK_ARG(dHall && dzall);
  const int Nb = (int)((L + E - 1) / E);
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(Nb, B * H);
  auto K = static_cast<const uint16_t*>(k);
  auto dK = static_cast<const uint16_t*>(dk);
  auto V = static_cast<const uint16_t*>(v);
  auto dV = static_cast<const uint16_t*>(dv);
  auto VT = static_cast<uint16_t*>(vt);
  auto KT = static_cast<uint16_t*>(kt);
  if (dtype == SLA2H_DTYPE_BF16) {
    if (tan)
      linear_states_kernel<BF16, true><<<grid, 256, 0, st>>>(K, dK, V, dV, L, Np, Nb, Hb, dHb, zb, dzb, VT, KT);
    else
      linear_states_kernel<BF16, false><<<grid, 256, 0, st>>>(K, dK, V, dV, L, Np, Nb, Hb, dHb, zb, dzb, VT, KT);
  } else {
    if (tan)
      linear_states_kernel<F16, true><<<grid, 256, 0, st>>>(K, dK, V, dV, L, Np, Nb, Hb, dHb, zb, dzb, VT, KT);
    else
      linear_states_kernel<F16, false><<<grid, 256, 0, st>>>(K, dK, V, dV, L, Np, Nb, Hb, dHb, zb, dzb, VT, KT);
  }
  int err = (int)hipGetLastError();
  if (err || Hall == nullptr) return err;
  dim3 g2(8320 / 64, B * H);
  states_sum_kernel<<<g2, 256, 0, st>>>(Hb, tan ? dHb : nullptr, zb, tan ? dzb : nullptr, Np, Hall,
                                        dHall, zall, dzall);
  return (int)hipGetLastError();
}

extern "C" int sla2h_linear_states_qat(const void* k, const void* v, int dtype, int B, int H,
                                       int64_t L, int D, int E, float* Hb, float* zb, float* Hall,
                                       float* zall, void* vt, void* stream) {
  SLA2H_CHECK_ARG(k && v && Hb && zb && Hall && zall);
  SLA2H_CHECK_ARG(D == kT && E == kT);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && B * H <= 65535 && L > 0);
  const int Nb = (int)((L + E - 1) / E);
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(Nb, B * H);
  auto K = static_cast<const uint16_t*>(k);
  auto V = static_cast<const uint16_t*>(v);
  if (dtype == SLA2H_DTYPE_BF16)
    linear_states_kernel<BF16, false, true><<<grid, 256, 0, st>>>(K, nullptr, V, nullptr, L, Nb, Nb, Hb, nullptr, zb, nullptr, static_cast<uint16_t*>(vt), nullptr);
  else
    linear_states_kernel<F16, false, true><<<grid, 256, 0, st>>>(K, nullptr, V, nullptr, L, Nb, Nb, Hb, nullptr, zb, nullptr, static_cast<uint16_t*>(vt), nullptr);
  int err = (int)hipGetLastError();
  if (err) return err;
  dim3 g2(8320 / 64, B * H);
  states_sum_kernel<<<g2, 256, 0, st>>>(Hb, nullptr, zb, nullptr, Nb, Hall, nullptr, zall, nullptr);
  return (int)hipGetLastError();
}

// Inference states of the 1-D SLA2 (_hblocks through complement_linear_states,
// models/sla2_vendor/kernel_linear.py:396-427, 496-504): phi(K) rounded to the
// 16-bit type, HALL_j = phi(K_j)^T V_j rounded to the 16-bit type (held as
// fp32 values), ZALL_j = colsum phi(K_j) in fp32, for every key block; the
// sums over the blocks when Hall / zall are given; the primal value operand
// tiles of the 16-bit sparse kernel when vt is given.
extern "C" int sla2h_hblocks_states(const void* k, const void* v, int dtype, int B, int H,
                                    int64_t L, int D, int E, float* Hb, float* zb, float* Hall,
                                    float* zall, void* vt, void* stream) {
  SLA2H_CHECK_ARG(k && v && Hb && zb);
  SLA2H_CHECK_ARG((Hall == nullptr) == (zall == nullptr));
  SLA2H_CHECK_ARG(D == kT && E == kT);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && B * H <= 65535 && L > 0);
  const int Nb = (int)((L + E - 1) / E);
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(Nb, B * H);
  auto K = static_cast<const uint16_t*>(k);
  auto V = static_cast<const uint16_t*>(v);
  if (dtype == SLA2H_DTYPE_BF16)
    linear_states_kernel<BF16, false, true, true><<<grid, 256, 0, st>>>(K, nullptr, V, nullptr, L, Nb, Nb, Hb, nullptr, zb, nullptr, static_cast<uint16_t*>(vt), nullptr);
  else
    linear_states_kernel<F16, false, true, true><<<grid, 256, 0, st>>>(K, nullptr, V, nullptr, L, Nb, Nb, Hb, nullptr, zb, nullptr, static_cast<uint16_t*>(vt), nullptr);
  int err = (int)hipGetLastError();
  if (err || Hall == nullptr) return err;
  dim3 g2(8320 / 64, B * H);
  states_sum_kernel<<<g2, 256, 0, st>>>(Hb, nullptr, zb, nullptr, Nb, Hall, nullptr, zall, nullptr);
  return (int)hipGetLastError();
}

// Backward complement.  sel[bh][n][kc] bit j = 1 where query block
// m = 32 kc + j routes tile n (augmented LUT); the GEMM above then runs with
// the roles swapped: rows = tiles n, contraction over query blocks m, mask
// = NOT sel, operands = the per-query-block partials [P | Pz].
__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

__global__ __launch_bounds__(256) void sel_scatter_kernel(const int32_t* __restrict__ lut, int Mb,
                                                         int Mq, int qshift, int J, int NCq,
                                                         uint32_t* __restrict__ sel) {
  const int bh = blockIdx.y;
  const int idx = blockIdx.x * 256 + threadIdx.x;  // over 64-row query blocks x J
  if (idx >= Mb * J) return;
  const int m = idx / J;
  const int n = lut[((int64_t)bh * Mq + (m >> qshift)) * J + (idx - m * J)];
  if ((unsigned)n < (unsigned)Mb)
    atomicOr(&sel[((int64_t)bh * Mb + n) * NCq + (m >> 5)], 1u << (m & 31));
}

__global__ __launch_bounds__(256) void sel_complement_kernel(const uint32_t* __restrict__ sel,
                                                            int Mb, int NCq, int MTp,
                                                            uint32_t* __restrict__ cbits) {
  const int bh = blockIdx.y;
  const int idx = blockIdx.x * 256 + threadIdx.x;  // over NCq * MTp
  if (idx >= NCq * MTp) return;
  const int kc = idx / MTp, n = idx - kc * MTp;
  uint32_t wd = 0u;
  if (n < Mb) {
    const int nv = Mb - 32 * kc;
    const uint32_t valid = nv >= 32 ? 0xffffffffu : ((1u << nv) - 1u);
    wd = ~sel[((int64_t)bh * Mb + n) * NCq + kc] & valid;
  }
  cbits[(int64_t)bh * NCq * MTp + idx] = wd;
}

extern "C" int sla2h_complement_bwd(const float* P, const float* Pz, const int32_t* lut_aug,
                                    int B, int H, int Mb, int bq, int J, void* workspace,
                                    uint32_t* sel, void* comp, void* stream) {
  SLA2H_CHECK_ARG(P && Pz && lut_aug && workspace && sel && comp);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && B * H <= 65535 && Mb > 0 && Mb <= 4096 && J >= 1);
  SLA2H_CHECK_ARG(bq == 64 || bq == 128 || bq == 256);
  const int qshift = bq == 64 ? 0 : (bq == 128 ? 1 : 2);
  const int Mq = (Mb + (1 << qshift) - 1) >> qshift;
  const int MT = (Mb + 15) / 16, NC = (Mb + 31) / 32;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nsel = (int64_t)B * H * Mb * NC;
  fill_u32_kernel<<<(unsigned)((nsel + 255) / 256), 256, 0, st>>>(sel, nsel);
  sel_scatter_kernel<<<dim3((Mb * J + 255) / 256, B * H), 256, 0, st>>>(lut_aug, Mb, Mq, qshift, J,
                                                                       NC, sel);
  auto cbits = static_cast<uint32_t*>(workspace);
  sel_complement_kernel<<<dim3((NC * MT * 16 + 255) / 256, B * H), 256, 0, st>>>(sel, Mb, NC,
                                                                               MT * 16, cbits);
  int err = (int)hipGetLastError();
  if (err) return err;
  dim3 grid(4160 / kCompCols, B * H, (MT + kMaskSub - 1) / kMaskSub);
  comp_gemm_kernel<false><<<grid, kCompThreads, 0, st>>>(P, nullptr, Pz, nullptr, cbits, Mb, Mb,
                                                         MT, NC, static_cast<unsigned char*>(comp));
  return (int)hipGetLastError();
}

extern "C" size_t sla2h_complement_workspace_bytes(int B, int H, int Mb, int Np) {
  if (B <= 0 || H <= 0 || Mb <= 0 || Np <= 0) return 0;
  const size_t MT = (size_t)(Mb + 15) / 16, NC = (size_t)(Np + 31) / 32;
  return (size_t)B * H * NC * MT * 16 * 4;
}

// ---------------------------------------------------------------------------
// Allocation-free complement: the bit-mask workspace lives in this file-scope
// device array (one copy per GPU, held until the process ends).  Host code
// never uses the array's name as an address: the device address of each GPU's
// copy comes from hipGetSymbolAddress, taken once per device on the first
// call with that device current, and is kept here.  The mask kernel writes
// every word the GEMM reads, so nothing needs clearing between calls; calls
// that overlap on one GPU (several streams or threads) race on the array.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[SLA2H_COMPLEMENT_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int complement_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (ptr == nullptr) return (int)hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}
}  // namespace

extern "C" int sla2h_complement(const float* Hb, const float* dHb, const float* zb,
                                const float* dzb, const int32_t* lut, int B, int H, int Mb,
                                int Np, int D, int T, void* workspace, void* comp,
                                void* stream) {
  SLA2H_CHECK_ARG(Hb && zb && lut && comp && workspace);
  SLA2H_CHECK_ARG(D == kT);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && B * H <= 65535 && Mb > 0 && Np > 0 && Np <= 4096);
  SLA2H_CHECK_ARG(T >= 1 && T <= Np);
  const bool tan = dHb != nullptr;
  if (tan) SLA2H_CHECK_ARG(dzb);
  const int MT = (Mb + 15) / 16, NC = (Np + 31) / 32;
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto cbits = static_cast<uint32_t*>(workspace);
  auto out = static_cast<unsigned char*>(comp);
  // mask bits plus the z parts of the records; the GEMM takes the H parts only
  // (128 or 64 column tiles per head: whole rounds of workgroups)
  comp_mask_kernel<<<dim3(MT, B * H), tan ? 512 : 256, (size_t)16 * NC * 4, st>>>(
      lut, Mb, Np, T, MT, NC, cbits, zb, dzb, out);
  int err = (int)hipGetLastError();
  if (err) return err;
  const int ncols = tan ? 8192 : 4096;
  dim3 grid(ncols / kCompCols, B * H, (MT + kMaskSub - 1) / kMaskSub);
  if (tan)
    comp_gemm_kernel<true><<<grid, kCompThreads, 0, st>>>(Hb, dHb, zb, dzb, cbits, Mb, Np, MT, NC, out);
  else
    comp_gemm_kernel<false><<<grid, kCompThreads, 0, st>>>(Hb, nullptr, zb, nullptr, cbits, Mb, Np, MT, NC, out);
  return (int)hipGetLastError();
}

extern "C" int sla2h_complement_noalloc(const float* Hb, const float* dHb, const float* zb,
                                        const float* dzb, const int32_t* lut, int B, int H,
                                        int Mb, int Np, int D, int T, void* comp, void* stream) {
  SLA2H_CHECK_ARG(Hb && zb && lut && comp);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && Mb > 0 && Np > 0);
  SLA2H_CHECK_ARG(sla2h_complement_workspace_bytes(B, H, Mb, Np) <=
                  (size_t)SLA2H_COMPLEMENT_SCRATCH_BYTES);
  void* ws = nullptr;
  const int err = complement_scratch(&ws);
  if (err) return err;
  return sla2h_complement(Hb, dHb, zb, dzb, lut, B, H, Mb, Np, D, T, ws, comp, stream);
}
