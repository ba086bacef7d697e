// Sparse branch of the SLA2 cube attention in the training-forward semantics
// of _attn_fwd_qat (models/sla2_vendor/kernel_sparse_qat.py:28-117, with
// USE_INT8, BLOCK_N = 64, PHI_OUT), gfx950:
//   S = int32(Q8 . K8^T) * (sq * sk) * scale * log2(e), keys past L masked;
//   running maximum m per block of keys (exact), P = exp2(S - m),
//   P8 = (int) fl(127 P + 0.5), O += int32(P8 . V8) * (sv / 127) after the
//   rescale of O and l by exp2(m_old - m); o_s = O / l (16-bit),
//   lse = m + log2(l) (fp32), and phi(Q) = softmax_D(Q) (16-bit).
// Q8, K8, V8 and their per-tile scales come from sla2h_quant_train (the
// reference quantises in-kernel with the same law; the result is the same).
//
// Work unit: one 64-row query block of one (b, h), one workgroup of 4 wave64;
// wave w owns queries 16w..16w+15 and all 64 keys of every tile.  Scores are
// computed transposed (S^T = K8 Q8^T, four 16-key blocks): a lane holds 16
// keys of one query, which is directly the B operand of the INT8 MFMA
// O^T = V8^T P8^T (K = 64 keys; V8 is stored in the matching fragment order).
// Key and value fragments are loaded one tile ahead.
#include "common.h"

#include <climits>
#include <type_traits>

namespace sla2h {

namespace {

constexpr int kT = 64;
constexpr int kMaxJ = 1024;

struct TrainArgs {
  const uint16_t* q;
  const int8_t* q8;
  const int8_t* k8;
  const int8_t* v8f;
  const float* qs;
  const float* ks;
  const float* vs;
  const int32_t* lut;
  uint16_t* os;
  float* lse;
  uint16_t* qphi;
  float* os32 = nullptr;  // set: o_s is written here in fp32 instead of os
  int64_t L;
  int Nb, Np, Mb, T, n_tail, nwork, per_xcd;
  int Mq, qshift;  // LUT rows: query blocks of 64 << qshift rows
  int Mqs, qsb;    // Q scales: blocks of 1 << qsb rows (per lane)
  float c2;        // fl32(scale * log2(e))
};

constexpr float kLog2_127 = 6.98868469f;  // log2(127)

template <typename T16>
__global__ __launch_bounds__(256, 2) void sparse_fwd_qat_kernel(TrainArgs a) {
  __shared__ int2 tiles[kMaxJ];  // (tile id, bits of sk)
  __shared__ float vsc[kMaxJ];   // sv / 127 of each visited tile
  // the visited key tile's K8 and V8 MFMA fragments, double-buffered: each
  // tile is fetched once per workgroup (wave w fetching fragment w of each)
  // and read by all four waves
  __shared__ __align__(16) i32x4 kfr[2][4][64];
  __shared__ __align__(16) i32x4 vfr[2][4][64];

  const int logical = (blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
  if (logical >= a.nwork) return;
  const int bh = __builtin_amdgcn_readfirstlane(logical / a.Mb);
  const int m = __builtin_amdgcn_readfirstlane(logical - bh * a.Mb);
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, r = l & 15, g = l >> 4;
  const int64_t L = a.L;
  const int64_t qkbase = (int64_t)bh * L;
  const int64_t qrow = (int64_t)m * kT + 16 * w + r;  // this lane's query
  const bool qok = qrow < L;

  const int J = a.T + a.n_tail;
  const int32_t* lrow = a.lut + ((int64_t)bh * a.Mq + (m >> a.qshift)) * a.T;
  for (int j = tid; j < J; j += 256) {
    int n = j < a.T ? lrow[j] : a.Np + (j - a.T);
    n = n < 0 ? 0 : (n >= a.Nb ? a.Nb - 1 : n);
    tiles[j] = make_int2(n, __builtin_bit_cast(int, a.ks[(int64_t)bh * a.Nb + n]));
    vsc[j] = a.vs[(int64_t)bh * a.Nb + n] / 127.0f;
  }

  // phi(Q) of this lane's 16 channels 16g..16g+15 (row max / sum over the
  // four lane groups), written as 16-bit
  {
    float x[16];
    uint4 u0 = make_uint4(0, 0, 0, 0), u1 = u0;
    if (qok) {
      const uint4* src = reinterpret_cast<const uint4*>(a.q + (qkbase + qrow) * kT + 16 * g);
      u0 = src[0];
      u1 = src[1];
    }
    const uint32_t wd[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[2 * i] = T16::to_f32((uint16_t)(wd[i] & 0xffff));
      x[2 * i + 1] = T16::to_f32((uint16_t)(wd[i] >> 16));
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, x[i]);
    mx = max_over_groups(mx);
    float den = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      x[i] = __expf(x[i] - mx);
      den += x[i];
    }
    den = sum_over_groups(den);
    const float rd = 1.f / den;
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = pack_pair<T16>(x[2 * i] * rd, x[2 * i + 1] * rd);
    if (qok && a.qphi != nullptr) {
      uint4* dst = reinterpret_cast<uint4*>(a.qphi + (qkbase + qrow) * kT + 16 * g);
      dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
      dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
  }
  __syncthreads();

  // INT8 Q B operand: this lane's query, channels 16g..16g+15
  const i32x4 q8f = qok ? *reinterpret_cast<const i32x4*>(a.q8 + (qkbase + qrow) * kT + 16 * g)
                        : i32x4{0, 0, 0, 0};
  const int qsi = (int)(qrow >> a.qsb);  // this lane's Q scale block
  const float sq = a.qs[(int64_t)bh * a.Mqs + (qsi < a.Mqs ? qsi : a.Mqs - 1)];
  const auto rk8 = make_rsrc(a.k8 + qkbase * kT, L * kT);  // key rows past L read as 0
  const auto rv8 = make_rsrc(a.v8f + (int64_t)bh * a.Nb * 4096, (int64_t)a.Nb * 4096);
  const int k8off = r * kT + 16 * g;  // + 16 kb rows + tile base

  struct Frags {
    i32x4 k[4];  // K8[16kb + r][16g ..]
    i32x4 v[4];  // V8 fragments of column tile ct
  };
  // wave w fetches K8 fragment w (keys 16w + r, channels 16g..16g+15) and V8
  // fragment w (column tile w) of tile j into registers ...
  auto gload = [&](int j, i32x4& kr, i32x4& vr) {
    const int n = __builtin_amdgcn_readfirstlane(tiles[j].x);
    kr = __builtin_bit_cast(i32x4, buf_load16(rk8, k8off + (n * kT + 16 * w) * kT, 0));
    vr = __builtin_bit_cast(i32x4, buf_load16(rv8, w * 1024 + l * 16, n * 4096));
  };
  // ... stores them in LDS slot s, and every wave reads all eight
  auto lstore = [&](int s, const i32x4& kr, const i32x4& vr) {
    kfr[s][w][l] = kr;
    vfr[s][w][l] = vr;
  };
  auto lread = [&](int s, Frags& f) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) f.k[kb] = kfr[s][kb][l];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) f.v[ct] = vfr[s][ct][l];
  };

  f32x4 acc[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) acc[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_i = -INFINITY, l_i = 0.f;  // l_i: this lane's 16 keys per tile, reduced at the end

  // MASK: the tile reaches past L (its keys there are masked); other tiles
  // skip the per-key test
  // Unmasked tiles (all but a ragged last one) spend about half the VALU work
  // per score of the reference's written steps:
  //  * the tile's row maximum comes from the integer scores: with c > 0 and
  //    monotonic rounding, max_j fl(s_j c) = fl(max_j s_j c), one v_max3 per
  //    two scores instead of a conversion, two products and a maximum each;
  //  * the exponent is one fma(s, c, -(m - log2 127)) with c = fl(sq sk
  //    scale log2 e), which gives 127 p directly (the reference rounds s sq
  //    sk, then the product by scale log2 e, then the difference, then p,
  //    then 127 p: the results differ by a few ulps of 127 p);
  //  * P8 = rne(127 p) by v_cvt_pk_u8_f32, which converts with round to
  //    nearest even and packs the byte in one instruction.  rne(127 p) equals
  //    trunc(127 p + 0.5) exactly: 127 p lies on a half-integer only for
  //    p = 1/2 (127 is odd and prime), where both give 64; the reference's
  //    trunc(fl(127 p + 0.5)) differs where that sum rounds up onto an
  //    integer (one entry in about 10^5);
  //  * l sums 127 p (divided by 127 once at the end).
  // The masked tail tile keeps the reference's rounding steps (its l term is
  // scaled by 127 once per tile).
  auto tile = [&](const Frags& f, int j, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int n = __builtin_amdgcn_readfirstlane(tiles[j].x);
    const float sqk = sq * __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(tiles[j].y));
    const int64_t key0 = (int64_t)n * kT + 4 * g;
    float s[16];
    float lm = -INFINITY;
    const float c = sqk * a.c2;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const i32x4 si = mfma_i8_16x16x64(f.k[kb], q8f, i32x4{0, 0, 0, 0});
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (MASK) {
          float x = ((float)si[i] * sqk) * a.c2;
          if (key0 + 16 * kb + i >= L) x = -INFINITY;
          s[4 * kb + i] = x;
          lm = fmaxf(lm, x);
        } else {
          const int v = si[i];
          s[4 * kb + i] = (float)v;
        }
      }
    }
    if (!MASK) {
      float smx = s[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) smx = fmaxf(smx, s[i]);
      lm = smx * c;
    }
    lm = max_over_groups(lm);
    const float mn = fmaxf(m_i, lm);
    const float alpha = fast_exp2(m_i - mn);  // 0 on the first tile (m_i = -inf)
    const float mn127 = mn - kLog2_127;       // exponent shift of 127 p
    float ls = 0.f;
    uint32_t pk[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      if (MASK) {
        uint32_t wd = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = fast_exp2(s[4 * kb + i] - mn);
          ls += p;
          wd |= ((uint32_t)(int)fmaf(p, 127.f, 0.5f)) << (8 * i);  // p in [0, 1]: 0..127
        }
        pk[kb] = wd;
        if (kb == 3) ls *= 127.f;  // l in units of p / 127, as on unmasked tiles
      } else {
        // p127 = 127 p from the exponent (one shift per tile), l summed in
        // units of p / 127, P8 = rne(p127) converted and packed in one
        // instruction per byte (v_cvt_pk_u8_f32 rounds to nearest even)
        uint32_t wd = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p127 = fast_exp2(fmaf(s[4 * kb + i], c, -mn127));
          ls += p127;
          wd = __builtin_amdgcn_cvt_pk_u8_f32(p127, i, wd);
        }
        pk[kb] = wd;
      }
    }
    l_i = l_i * alpha + ls;
    // the exact maximum moves on few tiles: where no lane's does (alpha == 1
    // everywhere) the rescale acc * alpha is the identity and is skipped
    if (__builtin_amdgcn_ballot_w64(mn != m_i) != 0) {
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[ct][i] = acc[ct][i] * alpha;
    }
    m_i = mn;
    const i32x4 p8 = i32x4{(int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3]};
    const float sv = vsc[j];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const i32x4 pv = mfma_i8_16x16x64(f.v[ct], p8, i32x4{0, 0, 0, 0});
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[ct][i] = fmaf((float)pv[i], sv, acc[ct][i]);
    }
  };
  auto tile_any = [&](const Frags& f, int j) {
    if ((int64_t)(__builtin_amdgcn_readfirstlane(tiles[j].x) + 1) * kT > L)
      tile(f, j, std::true_type{});
    else
      tile(f, j, std::false_type{});
  };

  // tile j in slot j & 1; tile j + 1 is fetched while tile j is computed and
  // stored after it (the slot was last read before the previous barrier)
  {
    i32x4 kr, vr;
    gload(0, kr, vr);
    lstore(0, kr, vr);
  }
  __syncthreads();
  for (int j = 0; j < J; ++j) {
    Frags f;
    lread(j & 1, f);
    i32x4 kr, vr;
    const bool more = j + 1 < J;
    if (more) gload(j + 1, kr, vr);
    tile_any(f, j);
    if (more) lstore((j + 1) & 1, kr, vr);
    __syncthreads();
  }

  const float lt = sum_over_groups(l_i) * (1.f / 127.f);  // l_i counts 127 p
  const float rl = 1.f / lt;
  // lane (g, r) holds O^T[16 ct + 4g + i][query r]
  if (qok) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int64_t oo = (qkbase + qrow) * kT + 16 * ct + 4 * g;
      if (a.os32 != nullptr) {
        *reinterpret_cast<f32x4*>(a.os32 + oo) =
            f32x4{acc[ct][0] * rl, acc[ct][1] * rl, acc[ct][2] * rl, acc[ct][3] * rl};
      } else {
        const uint32_t lo = pack_pair<T16>(acc[ct][0] * rl, acc[ct][1] * rl);
        const uint32_t hi = pack_pair<T16>(acc[ct][2] * rl, acc[ct][3] * rl);
        *reinterpret_cast<uint2*>(a.os + oo) = make_uint2(lo, hi);
      }
    }
    if (g == 0) a.lse[qkbase + qrow] = m_i + __log2f(lt);
  }
}

// 16-bit variant of the same recurrence (_attn_fwd_qat without USE_INT8,
// kernel_sparse_qat.py:28-117, as run by the 1-D SLA2 module): S = q.k^T on
// 16-bit MFMA (fp32 accumulate) * scale * log2(e), exact running maximum,
// O += round16(P) . V.  Query blocks of 64 << qshift rows share one LUT row;
// every key block is routable (the last one possibly partial).  Wave w owns
// queries 16w..16w+15 and all 64 keys of a tile: S^T = K Q^T leaves a lane
// with 16 keys of one query, which packed in pairs of 16-key groups is the B
// operand of O^T = V^T P^T on 16x16x32 (V^T from the primal vt operand tiles).
struct Fwd16Args {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;
  const int32_t* lut;
  uint16_t* os;
  float* lse;
  uint16_t* qphi;
  float* os32 = nullptr;  // set: o_s is written here in fp32 instead of os
  int64_t L;
  int Nb, Mq, qshift, T, nwork, per_xcd;
  float c;  // fl32(scale * log2(e))
};

template <typename T16>
__global__ __launch_bounds__(256, 2) void sparse_fwd16_kernel(Fwd16Args a) {
  __shared__ int tiles[kMaxJ];
  // the visited key tile's K and V^T MFMA fragments, double-buffered: each
  // tile is fetched once per workgroup (wave w fetching K rows 16w..16w+15 and
  // V^T column tile w) and read by all four waves
  __shared__ __align__(16) u32x4 ksh[2][4][2][64];  // [slot][kb][ks][lane]
  __shared__ __align__(16) u32x2 vsh[2][4][4][64];  // [slot][ct][w'][lane]

  const int logical = (blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
  if (logical >= a.nwork) return;
  const int bh = __builtin_amdgcn_readfirstlane(logical / a.Nb);
  const int m = __builtin_amdgcn_readfirstlane(logical - bh * a.Nb);
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, r = l & 15, g = l >> 4;
  const int64_t L = a.L;
  const int64_t qkbase = (int64_t)bh * L;
  const int64_t qrow = (int64_t)m * kT + 16 * w + r;
  const bool qok = qrow < L;

  const int32_t* lrow = a.lut + ((int64_t)bh * a.Mq + (m >> a.qshift)) * a.T;
  for (int j = tid; j < a.T; j += 256) {
    const int n = lrow[j];
    tiles[j] = n < 0 ? 0 : (n >= a.Nb ? a.Nb - 1 : n);
  }

  // phi(Q) of this lane's 16 channels 16g..16g+15, written as 16-bit
  {
    float x[16];
    uint4 u0 = make_uint4(0, 0, 0, 0), u1 = u0;
    if (qok) {
      const uint4* src = reinterpret_cast<const uint4*>(a.q + (qkbase + qrow) * kT + 16 * g);
      u0 = src[0];
      u1 = src[1];
    }
    const uint32_t wd[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[2 * i] = T16::to_f32((uint16_t)(wd[i] & 0xffff));
      x[2 * i + 1] = T16::to_f32((uint16_t)(wd[i] >> 16));
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, x[i]);
    mx = max_over_groups(mx);
    float den = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      x[i] = __expf(x[i] - mx);
      den += x[i];
    }
    den = sum_over_groups(den);
    const float rd = 1.f / den;
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = pack_pair<T16>(x[2 * i] * rd, x[2 * i + 1] * rd);
    if (qok) {
      uint4* dst = reinterpret_cast<uint4*>(a.qphi + (qkbase + qrow) * kT + 16 * g);
      dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
      dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
  }
  // 16-bit Q B operand: this lane's query, channels 32ks + 8g .. +7
  u32x4 qf[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    qf[ks] = qok ? *reinterpret_cast<const u32x4*>(a.q + (qkbase + qrow) * kT + 32 * ks + 8 * g)
                 : u32x4{0, 0, 0, 0};
  __syncthreads();

  const auto rk = make_rsrc(a.k + qkbase * kT, L * kT * 2);  // key rows past L read as 0
  const auto rv = make_rsrc(a.vt + (int64_t)bh * a.Nb * 4096, (int64_t)a.Nb * 8192);
  struct Frags {
    u32x4 k[4][2];  // K[16kb + r][32ks + 8g ..]
    u32x2 v[4][4];  // [ct][w'] = V[16w' + 4g + 0..3][16ct + r]
  };
  // wave w fetches K fragment kb = w (both ks) and the 2 KB of V^T column tile
  // ct = w (32 contiguous bytes per lane) into registers ...
  struct Stage {
    u32x4 k[2];
    u32x4 v[2];
  };
  auto gload = [&](int j, Stage& st) {
    const int n = __builtin_amdgcn_readfirstlane(tiles[j]);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      st.k[ks] = buf_load16(rk, n * 8192 + ((16 * w + r) * kT + 32 * ks + 8 * g) * 2, 0);
#pragma unroll
    for (int h = 0; h < 2; ++h) st.v[h] = buf_load16(rv, w * 2048 + l * 32 + 16 * h, n * 8192);
  };
  // ... stores them in LDS slot sl (the same layout as in global memory for
  // V^T), and every wave reads the whole tile's fragments
  auto lstore = [&](int sl, const Stage& st) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) ksh[sl][w][ks][l] = st.k[ks];
    u32x4* vd = reinterpret_cast<u32x4*>(&vsh[sl][w][0][0]);
    vd[2 * l] = st.v[0];
    vd[2 * l + 1] = st.v[1];
  };
  auto lread = [&](int sl, Frags& f) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) f.k[kb][ks] = ksh[sl][kb][ks][l];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) f.v[ct][ww] = vsh[sl][ct][ww][l];
  };

  f32x4 acc[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) acc[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_i = -INFINITY, l_i = 0.f;

  // MASK as in sparse_fwd_qat_kernel: only a tile reaching past L tests keys
  auto tile = [&](const Frags& f, int j, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int n = __builtin_amdgcn_readfirstlane(tiles[j]);
    const int64_t key0 = (int64_t)n * kT + 4 * g;
    float s[16];
    float lm = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4 sc = mfma_16x16x32<T16>(f.k[kb][0], qf[0], f32x4{0.f, 0.f, 0.f, 0.f});
      sc = mfma_16x16x32<T16>(f.k[kb][1], qf[1], sc);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = sc[i] * a.c;
        if (MASK && key0 + 16 * kb + i >= L) x = -INFINITY;
        s[4 * kb + i] = x;
        lm = fmaxf(lm, x);
      }
    }
    lm = max_over_groups(lm);
    const float mn = fmaxf(m_i, lm);
    const float alpha = fast_exp2(m_i - mn);
    float ls = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      s[i] = fast_exp2(s[i] - mn);
      ls += s[i];
    }
    l_i = l_i * alpha + ls;
    // alpha == 1 on every lane (no maximum moved) leaves acc unchanged
    if (__builtin_amdgcn_ballot_w64(mn != m_i) != 0) {
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) acc[ct] *= alpha;
    }
    m_i = mn;
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const u32x4 pb = u32x4{pack_pair<T16>(s[8 * pp], s[8 * pp + 1]),
                             pack_pair<T16>(s[8 * pp + 2], s[8 * pp + 3]),
                             pack_pair<T16>(s[8 * pp + 4], s[8 * pp + 5]),
                             pack_pair<T16>(s[8 * pp + 6], s[8 * pp + 7])};
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const u32x4 av = u32x4{f.v[ct][2 * pp].x, f.v[ct][2 * pp].y, f.v[ct][2 * pp + 1].x,
                               f.v[ct][2 * pp + 1].y};
        acc[ct] = mfma_16x16x32<T16>(av, pb, acc[ct]);
      }
    }
  };
  auto tile_any = [&](const Frags& f, int j) {
    if ((int64_t)(__builtin_amdgcn_readfirstlane(tiles[j]) + 1) * kT > L)
      tile(f, j, std::true_type{});
    else
      tile(f, j, std::false_type{});
  };

  // tile j in slot j & 1; tile j + 1 is fetched while tile j is computed and
  // stored after it (the slot was last read before the previous barrier)
  const int J = a.T;
  {
    Stage st;
    gload(0, st);
    lstore(0, st);
  }
  __syncthreads();
  for (int j = 0; j < J; ++j) {
    Frags f;
    lread(j & 1, f);
    Stage st;
    const bool more = j + 1 < J;
    if (more) gload(j + 1, st);
    tile_any(f, j);
    if (more) lstore((j + 1) & 1, st);
    __syncthreads();
  }

  const float lt = sum_over_groups(l_i);
  const float rl = 1.f / lt;
  if (qok) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int64_t oo = (qkbase + qrow) * kT + 16 * ct + 4 * g;
      if (a.os32 != nullptr) {
        *reinterpret_cast<f32x4*>(a.os32 + oo) =
            f32x4{acc[ct][0] * rl, acc[ct][1] * rl, acc[ct][2] * rl, acc[ct][3] * rl};
      } else {
        const uint32_t lo = pack_pair<T16>(acc[ct][0] * rl, acc[ct][1] * rl);
        const uint32_t hi = pack_pair<T16>(acc[ct][2] * rl, acc[ct][3] * rl);
        *reinterpret_cast<uint2*>(a.os + oo) = make_uint2(lo, hi);
      }
    }
    if (g == 0) a.lse[qkbase + qrow] = m_i + __log2f(lt);
  }
}

// Linear branch and mix of the training forward (_lin_fwd2 in its state form,
// models/sla2_vendor/kernel_linear.py:274-304, and the mix at
// models/sla2_cube_qat.py:742-744), one 64-row query block per workgroup:
//   H_i = htot16 - sum_{j in lut_aug(i)} phi(K_j)^T V_j, rounded to 16 bits,
//   num = phi(Q) H_i (16-bit MFMA, fp32 accumulate), den = phi(Q) . z_i +- eps,
//   o_l = num / den, o = a o_s + (1 - a) o_l with every product, difference
//   and sum rounded to the 16-bit type as the reference's half-precision
//   tensor arithmetic does.
// The complement record holds sum over the tiles NOT in lut_aug of
// phi(K_j)^T V_j; H_i = record + (htot16 - htot) with htot = sum over all tiles
// (the same sum, in another fp32 order).  Wave w owns queries 16w..16w+15;
// lane (g, r) holds query r, output channels 16 ct + 4g + i.
constexpr int kRecH = 0, kRecZ = 32768, kRecBytes = 33280;

// INFER: the inference law of _lin_fwd3 (models/sla2_vendor/kernel_linear.py:
// 446-493): H_i = the complement record itself (a sum of 16-bit block
// states), rounded to the 16-bit type for the product; o_l and the mix stay
// fp32 (o = a o_s + (1 - a) o_l, one rounding at the store); Hall, o_l and
// den_out may be null.
template <typename T16, bool INFER = false>
__global__ __launch_bounds__(256) void linear_mix_qat_kernel(
    const uint16_t* __restrict__ qphi, const unsigned char* __restrict__ comp,
    const float* __restrict__ Hall, const uint16_t* __restrict__ o_s,
    const float* __restrict__ alpha, int alpha_stride, int64_t L, int Mq, int qshift, int H,
    float eps_l, uint16_t* __restrict__ o, uint16_t* __restrict__ o_l, float* __restrict__ den_out) {
  __shared__ __align__(16) uint16_t hT[kT][kT + 8];  // [value channel][key channel]
  __shared__ float zs[kT];

  const int m = blockIdx.x, bh = blockIdx.y, h = bh % H;
  const int mq = m >> qshift;  // record and alpha of this 64-row block's query block
  const int tid = threadIdx.x;
  const unsigned char* rec = comp + ((int64_t)bh * Mq + mq) * kRecBytes;
  {
    const int d = tid >> 2, v0 = (tid & 3) * 16;
    const f32x4* hr = reinterpret_cast<const f32x4*>(rec + kRecH) + (d * kT + v0) / 4;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const f32x4 x = hr[c];
      if (INFER) {
#pragma unroll
        for (int i = 0; i < 4; ++i) hT[v0 + 4 * c + i][d] = T16::from_f32(x[i]);
      } else {
        const f32x4 t = reinterpret_cast<const f32x4*>(Hall + (int64_t)bh * kT * kT + d * kT + v0)[c];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float t16 = T16::to_f32(T16::from_f32(t[i]));
          hT[v0 + 4 * c + i][d] = T16::from_f32(x[i] + (t16 - t[i]));
        }
      }
    }
    if (tid < kT) zs[tid] = reinterpret_cast<const float*>(rec + kRecZ)[tid];
  }
  __syncthreads();

  const int w = tid >> 6, l = tid & 63, r = l & 15, g = l >> 4;
  const int64_t qrow = (int64_t)m * kT + 16 * w + r;
  const bool qok = qrow < L;
  const int64_t rowoff = ((int64_t)bh * L + qrow) * kT;
  u32x4 qb[2];
  float dn = 0.f;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    qb[ks] = qok ? *reinterpret_cast<const u32x4*>(qphi + rowoff + 32 * ks + 8 * g)
                 : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dn += T16::to_f32((uint16_t)(qb[ks][e] & 0xffff)) * zs[32 * ks + 8 * g + 2 * e];
      dn += T16::to_f32((uint16_t)(qb[ks][e] >> 16)) * zs[32 * ks + 8 * g + 2 * e + 1];
    }
  }
  dn = sum_over_groups(dn);
  dn = dn >= 0.f ? dn + eps_l : dn - eps_l;
  const float rdn = 1.f / dn;
  const float af = alpha[(int64_t)h * alpha_stride + mq];
  const float a16 = INFER ? af : T16::to_f32(T16::from_f32(af));
  const float b16 = INFER ? 1.f - af : T16::to_f32(T16::from_f32(1.f - a16));
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    f32x4 num = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x4 av = *reinterpret_cast<const u32x4*>(&hT[16 * ct + r][32 * ks + 8 * g]);
      num = mfma_16x16x32<T16>(av, qb[ks], num);
    }
    if (qok) {
      const int64_t oo = rowoff + 16 * ct + 4 * g;
      const uint2 sv = *reinterpret_cast<const uint2*>(o_s + oo);
      const uint32_t sw[2] = {sv.x, sv.y};
      float ol[4], ov[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float os16 = T16::to_f32((uint16_t)(sw[i >> 1] >> (16 * (i & 1))));
        if (INFER) {
          ol[i] = num[i] * rdn;
          ov[i] = a16 * os16 + b16 * ol[i];
        } else {
          ol[i] = T16::to_f32(T16::from_f32(num[i] * rdn));
          const float x = T16::to_f32(T16::from_f32(a16 * os16));
          const float y = T16::to_f32(T16::from_f32(b16 * ol[i]));
          ov[i] = x + y;
        }
      }
      *reinterpret_cast<uint2*>(o + oo) =
          make_uint2(pack_pair<T16>(ov[0], ov[1]), pack_pair<T16>(ov[2], ov[3]));
      if (o_l != nullptr)
        *reinterpret_cast<uint2*>(o_l + oo) =
            make_uint2(pack_pair<T16>(ol[0], ol[1]), pack_pair<T16>(ol[2], ol[3]));
    }
  }
  if (qok && g == 0 && den_out != nullptr) den_out[(int64_t)bh * L + qrow] = dn;
}

// Score form of the same linear branch (_lin_fwd2 with SCORE_FORM,
// models/sla2_vendor/kernel_linear.py:260-272), which the reference selects
// while the augmented LUT has at most 4 columns: the routed tiles are
// subtracted in the score domain instead of from the state,
//   num = qphi round16(Hall) - sum_j round16(W_j) V_j,  W_j = qphi kphi_j^T (fp32),
//   den = qphi . zall - sum_j rowsum(W_j), then +-eps_l (signed),
// kphi_j = round16(softmax_D(K rows of tile j)), zero past L.  The mix is
// linear_mix_qat_kernel's.  Wave w owns queries 16w..16w+15 and computes
// W^T = kphi_j qphi^T, so lane (g, r) holds keys 16 kt + 4g + i of query r.
// Those 8 keys of key tiles 2ks, 2ks+1 are directly the B operand of
// num^T -= V_j^T round16(W^T) for contraction chunk ks, with the K slot
// 8g + e standing for key 16 (2ks + e/4) + 4g + e%4; the A operand V_j^T is
// read from LDS in that key order.  Tile ids outside [0, Nb) are clamped.
// FUSED: the mix of the fused Algorithm-2 kernel (models/sla2_vendor/
// kernel_fused.py:116-124): o_s is fp32, o = a o_s + (1 - a) num / den in
// fp32 with alpha unrounded, one rounding at the store; o_l and den are not
// written.
template <typename T16, bool FUSED = false>
__global__ __launch_bounds__(256) void linear_mix_score_kernel(
    const uint16_t* __restrict__ qphi, const uint16_t* __restrict__ K,
    const uint16_t* __restrict__ V, const float* __restrict__ Hall,
    const float* __restrict__ zall, const int32_t* __restrict__ lut, int J, int Nb,
    const void* __restrict__ o_s, const float* __restrict__ alpha, int alpha_stride,
    int64_t L, int Mq, int qshift, int H, float eps_l, uint16_t* __restrict__ o,
    uint16_t* __restrict__ o_l, float* __restrict__ den_out) {
  __shared__ __align__(16) uint16_t hT[kT][kT + 8];  // round16(Hall)^T [value ch][key ch]
  __shared__ __align__(16) uint16_t kp[kT][kT + 8];  // kphi_j [key][ch]
  __shared__ __align__(16) uint16_t vT[kT][kT + 8];  // V_j^T [value ch][key]
  __shared__ float zs[kT];

  const int m = blockIdx.x, bh = blockIdx.y, h = bh % H;
  const int mq = m >> qshift;
  const int tid = threadIdx.x;
  {
    const int d = tid >> 2, v0 = (tid & 3) * 16;
    const f32x4* hr = reinterpret_cast<const f32x4*>(Hall + (int64_t)bh * kT * kT + d * kT + v0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const f32x4 x = hr[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) hT[v0 + 4 * c + i][d] = T16::from_f32(x[i]);
    }
    if (tid < kT) zs[tid] = zall[(int64_t)bh * kT + tid];
  }
  __syncthreads();

  const int w = tid >> 6, l = tid & 63, r = l & 15, g = l >> 4;
  const int64_t qrow = (int64_t)m * kT + 16 * w + r;
  const bool qok = qrow < L;
  const int64_t rowoff = ((int64_t)bh * L + qrow) * kT;
  u32x4 qb[2];
  float dn = 0.f;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    qb[ks] = qok ? *reinterpret_cast<const u32x4*>(qphi + rowoff + 32 * ks + 8 * g)
                 : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dn += T16::to_f32((uint16_t)(qb[ks][e] & 0xffff)) * zs[32 * ks + 8 * g + 2 * e];
      dn += T16::to_f32((uint16_t)(qb[ks][e] >> 16)) * zs[32 * ks + 8 * g + 2 * e + 1];
    }
  }
  dn = sum_over_groups(dn);
  f32x4 num[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    num[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x4 av = *reinterpret_cast<const u32x4*>(&hT[16 * ct + r][32 * ks + 8 * g]);
      num[ct] = mfma_16x16x32<T16>(av, qb[ks], num[ct]);
    }
  }

  // staging: thread (row sr, 16 channels from c0) of each selected tile
  const int sr = tid >> 2, c0 = (tid & 3) * 16;
  const int32_t* lrow = lut + ((int64_t)bh * Mq + mq) * J;
  float wsum = 0.f;  // this lane's keys of every tile, summed
  for (int j = 0; j < J; ++j) {
    const int n = min(max(lrow[j], 0), Nb - 1);
    const int64_t krow = (int64_t)n * kT + sr;
    const bool kok = krow < L;
    const int64_t koff = ((int64_t)bh * L + krow) * kT + c0;
    uint32_t kw[8], vw[8];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint4 ku = kok ? reinterpret_cast<const uint4*>(K + koff)[i] : make_uint4(0, 0, 0, 0);
      const uint4 vu = kok ? reinterpret_cast<const uint4*>(V + koff)[i] : make_uint4(0, 0, 0, 0);
      kw[4 * i + 0] = ku.x; kw[4 * i + 1] = ku.y; kw[4 * i + 2] = ku.z; kw[4 * i + 3] = ku.w;
      vw[4 * i + 0] = vu.x; vw[4 * i + 1] = vu.y; vw[4 * i + 2] = vu.z; vw[4 * i + 3] = vu.w;
    }
    float x[16];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      x[i] = T16::to_f32((uint16_t)(kw[i >> 1] >> (16 * (i & 1))));
      mx = fmaxf(mx, x[i]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      x[i] = __expf(x[i] - mx);
      sum += x[i];
    }
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    __syncthreads();  // the previous tile's kp / vT reads are done
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t p = kok ? pack_pair<T16>(x[2 * i] / sum, x[2 * i + 1] / sum) : 0u;
      *reinterpret_cast<uint32_t*>(&kp[sr][c0 + 2 * i]) = p;
      vT[c0 + 2 * i][sr] = (uint16_t)(vw[i] & 0xffff);
      vT[c0 + 2 * i + 1][sr] = (uint16_t)(vw[i] >> 16);
    }
    __syncthreads();

    f32x4 wt[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      wt[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const u32x4 av = *reinterpret_cast<const u32x4*>(&kp[16 * kt + r][32 * ks + 8 * g]);
        wt[kt] = mfma_16x16x32<T16>(av, qb[ks], wt[kt]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) wsum += wt[kt][i];
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const f32x4 a0 = wt[2 * ks], a1 = wt[2 * ks + 1];
      const u32x4 bw = u32x4{pack_pair<T16>(-a0[0], -a0[1]), pack_pair<T16>(-a0[2], -a0[3]),
                             pack_pair<T16>(-a1[0], -a1[1]), pack_pair<T16>(-a1[2], -a1[3])};
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const u32x2 v0 = *reinterpret_cast<const u32x2*>(&vT[16 * ct + r][32 * ks + 4 * g]);
        const u32x2 v1 = *reinterpret_cast<const u32x2*>(&vT[16 * ct + r][32 * ks + 16 + 4 * g]);
        num[ct] = mfma_16x16x32<T16>(u32x4{v0.x, v0.y, v1.x, v1.y}, bw, num[ct]);
      }
    }
  }
  dn -= sum_over_groups(wsum);
  dn = dn >= 0.f ? dn + eps_l : dn - eps_l;
  const float rdn = 1.f / dn;
  const float af = alpha[(int64_t)h * alpha_stride + mq];
  if (FUSED) {
    if (qok) {
      const float* os32 = static_cast<const float*>(o_s);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int64_t oo = rowoff + 16 * ct + 4 * g;
        const f32x4 sv = *reinterpret_cast<const f32x4*>(os32 + oo);
        float ov[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ov[i] = af * sv[i] + (1.f - af) * (num[ct][i] / dn);
        *reinterpret_cast<uint2*>(o + oo) =
            make_uint2(pack_pair<T16>(ov[0], ov[1]), pack_pair<T16>(ov[2], ov[3]));
      }
    }
    return;
  }
  const float a16 = T16::to_f32(T16::from_f32(af));
  const float b16 = T16::to_f32(T16::from_f32(1.f - a16));
  if (qok) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int64_t oo = rowoff + 16 * ct + 4 * g;
      const uint2 sv = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(o_s) + oo);
      const uint32_t sw[2] = {sv.x, sv.y};
      float ol[4], ov[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float os16 = T16::to_f32((uint16_t)(sw[i >> 1] >> (16 * (i & 1))));
        ol[i] = T16::to_f32(T16::from_f32(num[ct][i] * rdn));
        const float x = T16::to_f32(T16::from_f32(a16 * os16));
        const float y = T16::to_f32(T16::from_f32(b16 * ol[i]));
        ov[i] = x + y;
      }
      *reinterpret_cast<uint2*>(o + oo) =
          make_uint2(pack_pair<T16>(ov[0], ov[1]), pack_pair<T16>(ov[2], ov[3]));
      *reinterpret_cast<uint2*>(o_l + oo) =
          make_uint2(pack_pair<T16>(ol[0], ol[1]), pack_pair<T16>(ol[2], ol[3]));
    }
    if (g == 0) den_out[(int64_t)bh * L + qrow] = dn;
  }
}

}  // namespace

}  // namespace sla2h

using namespace sla2h;

extern "C" int sla2h_sparse_fwd_qat(const void* q, const int8_t* q8, const float* qs,
                                    const int8_t* k8, const float* ks, const int8_t* v8f,
                                    const float* vs, const int32_t* lut, int dtype, int B, int H,
                                    int64_t L, int D, int E, int Np, int T, float scale,
                                    void* o_s, float* lse, void* qphi, void* stream) {
  SLA2H_CHECK_ARG(q && q8 && qs && k8 && ks && v8f && vs && lut && o_s && lse && qphi);
  SLA2H_CHECK_ARG(D == kT && E == kT);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && L > 0 && Np > 0 && (int64_t)Np * E <= L);
  SLA2H_CHECK_ARG(T >= 1 && T <= Np);
  const int Nb = (int)((L + E - 1) / E);
  SLA2H_CHECK_ARG(T + (Nb - Np) <= kMaxJ);
  const int64_t nwork = (int64_t)Nb * B * H;
  const int64_t per_xcd = (nwork + 7) / 8;
  SLA2H_CHECK_ARG(8 * per_xcd < (1ll << 31));
  TrainArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q8 = q8;
  a.k8 = k8;
  a.v8f = v8f;
  a.qs = qs;
  a.ks = ks;
  a.vs = vs;
  a.lut = lut;
  a.os = static_cast<uint16_t*>(o_s);
  a.lse = lse;
  a.qphi = static_cast<uint16_t*>(qphi);
  a.L = L;
  a.Nb = Nb;
  a.Np = Np;
  a.Mb = Nb;
  a.T = T;
  a.n_tail = Nb - Np;
  a.Mq = Nb;
  a.qshift = 0;
  a.Mqs = Nb;
  a.qsb = 6;
  a.nwork = (int)nwork;
  a.per_xcd = (int)per_xcd;
  a.c2 = scale * 1.4426950408889634f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nblocks = (int)(8 * per_xcd);
  if (dtype == SLA2H_DTYPE_BF16)
    sparse_fwd_qat_kernel<BF16><<<nblocks, 256, 0, st>>>(a);
  else
    sparse_fwd_qat_kernel<F16><<<nblocks, 256, 0, st>>>(a);
  return (int)hipGetLastError();
}

static int log2_exact(int x) {
  int k = 0;
  while ((1 << k) < x) ++k;
  return (1 << k) == x ? k : -1;
}

// Inference INT8 sparse branch of the 1-D SLA2 (_attn_fwd_int8 through
// sparse_attention_int8, models/sla2_vendor/kernel_sparse_qat.py:154-247; the
// INT8 branch of _sla2_fwd_fused, kernel_fused.py:81-106): the same
// recurrence as above over every routable key block (the last one possibly
// partial), LUT rows per query block of bq rows, Q scales per block of
// qblock rows (bq for the unfused path, block_m for the fused one).
extern "C" int sla2h_sparse_fwd_int8(const void* q, const int8_t* q8, const float* qs, int qblock,
                                     const int8_t* k8, const float* ks, const int8_t* v8f,
                                     const float* vs, const int32_t* lut, int dtype, int B, int H,
                                     int64_t L, int D, int bq, int T, float scale, void* o_s,
                                     float* lse, void* qphi, void* stream) {
  SLA2H_CHECK_ARG(q && q8 && qs && k8 && ks && v8f && vs && lut && o_s && lse);
  SLA2H_CHECK_ARG(D == kT && (bq == 64 || bq == 128 || bq == 256));
  SLA2H_CHECK_ARG(qblock == 32 || qblock == 64 || qblock == 128 || qblock == 256);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && L > 0);
  const int Nb = (int)((L + kT - 1) / kT);
  SLA2H_CHECK_ARG(T >= 1 && T <= Nb && T <= kMaxJ);
  const int64_t nwork = (int64_t)Nb * B * H;
  const int64_t per_xcd = (nwork + 7) / 8;
  SLA2H_CHECK_ARG(8 * per_xcd < (1ll << 31));
  TrainArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q8 = q8;
  a.k8 = k8;
  a.v8f = v8f;
  a.qs = qs;
  a.ks = ks;
  a.vs = vs;
  a.lut = lut;
  a.os = static_cast<uint16_t*>(o_s);
  a.lse = lse;
  a.qphi = static_cast<uint16_t*>(qphi);
  a.L = L;
  a.Nb = Nb;
  a.Np = Nb;
  a.Mb = Nb;
  a.T = T;
  a.n_tail = 0;
  a.Mq = (int)((L + bq - 1) / bq);
  a.qshift = log2_exact(bq / kT);
  a.Mqs = (int)((L + qblock - 1) / qblock);
  a.qsb = log2_exact(qblock);
  a.nwork = (int)nwork;
  a.per_xcd = (int)per_xcd;
  a.c2 = scale * 1.4426950408889634f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nblocks = (int)(8 * per_xcd);
  if (dtype == SLA2H_DTYPE_BF16)
    sparse_fwd_qat_kernel<BF16><<<nblocks, 256, 0, st>>>(a);
  else
    sparse_fwd_qat_kernel<F16><<<nblocks, 256, 0, st>>>(a);
  return (int)hipGetLastError();
}

extern "C" int sla2h_linear_mix_qat(const void* qphi, const void* comp, const float* Hall,
                                    const void* o_s, const float* alpha, int alpha_stride,
                                    int dtype, int B, int H, int64_t L, int D, int E, float eps_l,
                                    void* o, void* o_l, float* den, void* stream) {
  SLA2H_CHECK_ARG(qphi && comp && Hall && o_s && alpha && o && o_l && den);
  SLA2H_CHECK_ARG(D == kT && (E == 64 || E == 128 || E == 256) && alpha_stride >= 0);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && B * H <= 65535 && L > 0);
  const int Mb = (int)((L + kT - 1) / kT);  // 64-row blocks
  const int Mq = (int)((L + E - 1) / E);     // query blocks of E rows (records, alpha)
  const int qshift = E == 64 ? 0 : (E == 128 ? 1 : 2);
  dim3 grid(Mb, B * H);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto QP = static_cast<const uint16_t*>(qphi);
  auto C = static_cast<const unsigned char*>(comp);
  auto OS = static_cast<const uint16_t*>(o_s);
  auto O = static_cast<uint16_t*>(o);
  auto OL = static_cast<uint16_t*>(o_l);
  if (dtype == SLA2H_DTYPE_BF16)
    linear_mix_qat_kernel<BF16><<<grid, 256, 0, st>>>(QP, C, Hall, OS, alpha, alpha_stride, L, Mq, qshift, H, eps_l, O, OL, den);
  else
    linear_mix_qat_kernel<F16><<<grid, 256, 0, st>>>(QP, C, Hall, OS, alpha, alpha_stride, L, Mq, qshift, H, eps_l, O, OL, den);
  return (int)hipGetLastError();
}

extern "C" int sla2h_linear_mix_score(const void* qphi, const void* k, const void* v,
                                      const float* Hall, const float* zall, const int32_t* lut,
                                      int J, const void* o_s, const float* alpha,
                                      int alpha_stride, int dtype, int B, int H, int64_t L, int D,
                                      int E, float eps_l, void* o, void* o_l, float* den,
                                      void* stream) {
  SLA2H_CHECK_ARG(qphi && k && v && Hall && zall && lut && o_s && alpha && o && o_l && den);
  SLA2H_CHECK_ARG(D == kT && (E == 64 || E == 128 || E == 256) && alpha_stride >= 0);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && B * H <= 65535 && L > 0 && J >= 1 && J <= kMaxJ);
  const int Nb = (int)((L + kT - 1) / kT);
  const int Mq = (int)((L + E - 1) / E);
  const int qshift = E == 64 ? 0 : (E == 128 ? 1 : 2);
  dim3 grid(Nb, B * H);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto QP = static_cast<const uint16_t*>(qphi);
  auto Kp = static_cast<const uint16_t*>(k);
  auto Vp = static_cast<const uint16_t*>(v);
  auto OS = static_cast<const uint16_t*>(o_s);
  auto O = static_cast<uint16_t*>(o);
  auto OL = static_cast<uint16_t*>(o_l);
  if (dtype == SLA2H_DTYPE_BF16)
    linear_mix_score_kernel<BF16><<<grid, 256, 0, st>>>(QP, Kp, Vp, Hall, zall, lut, J, Nb, OS, alpha, alpha_stride, L, Mq, qshift, H, eps_l, O, OL, den);
  else
    linear_mix_score_kernel<F16><<<grid, 256, 0, st>>>(QP, Kp, Vp, Hall, zall, lut, J, Nb, OS, alpha, alpha_stride, L, Mq, qshift, H, eps_l, O, OL, den);
  return (int)hipGetLastError();
}

extern "C" size_t sla2h_sla2_fused_workspace_bytes(int B, int H, int64_t L, int D) {
  if (B <= 0 || H <= 0 || L <= 0 || D != kT) return 0;
  const size_t rows = (size_t)B * H * L;
  const size_t os32 = (rows * kT * 4 + 255) / 256 * 256, qphi = (rows * kT * 2 + 255) / 256 * 256;
  return os32 + qphi + rows * 4;
}

// Fused SLA2 inference forward with the arithmetic of the fused Algorithm-2
// kernel (_sla2_fwd_fused, models/sla2_vendor/kernel_fused.py:29-124): the
// sparse branch (INT8 with Q scales per block_m rows, or 16-bit) writes o_s
// in fp32 to the workspace, then the score-form linear branch against the
// whole-sequence state and the fp32 mix produce o.  Two launches on one
// stream; the workspace holds o_s, phi(Q) and the row statistics.
extern "C" int sla2h_sla2_forward_fused(
    const void* q, const void* k, const void* v, const int8_t* q8, const float* qs, int block_m,
    const int8_t* k8, const float* ks, const int8_t* v8f, const float* vs, const void* vt,
    const float* Hall, const float* zall, const int32_t* lut, int T, const float* alpha,
    int alpha_stride, int dtype, int B, int H, int64_t L, int D, int bq, float scale,
    float eps_l, void* workspace, void* o, void* stream) {
  const bool int8 = q8 != nullptr;
  SLA2H_CHECK_ARG(q && k && v && Hall && zall && lut && alpha && workspace && o);
  SLA2H_CHECK_ARG(int8 ? (qs && k8 && ks && v8f && vs) : (vt != nullptr));
  SLA2H_CHECK_ARG(D == kT && (bq == 64 || bq == 128 || bq == 256) && alpha_stride >= 0);
  SLA2H_CHECK_ARG(!int8 || ((block_m == 32 || block_m == 64 || block_m == 128 || block_m == 256) &&
                            bq % block_m == 0));
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && B * H <= 65535 && L > 0 && L * kT * 2 < (1ll << 31));
  const int Nb = (int)((L + kT - 1) / kT);
  SLA2H_CHECK_ARG(T >= 1 && T <= Nb && T <= kMaxJ);
  const int64_t nwork = (int64_t)Nb * B * H;
  const int64_t per_xcd = (nwork + 7) / 8;
  SLA2H_CHECK_ARG(8 * per_xcd < (1ll << 31));
  const size_t rows = (size_t)B * H * L;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  float* os32 = reinterpret_cast<float*>(ws);
  uint16_t* qphi = reinterpret_cast<uint16_t*>(ws + (rows * kT * 4 + 255) / 256 * 256);
  float* lse = reinterpret_cast<float*>(ws + (rows * kT * 4 + 255) / 256 * 256 +
                                        (rows * kT * 2 + 255) / 256 * 256);
  const int Mq = (int)((L + bq - 1) / bq);
  const int qshift = bq == 64 ? 0 : (bq == 128 ? 1 : 2);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nblocks = (int)(8 * per_xcd);
  const bool bf = dtype == SLA2H_DTYPE_BF16;
  if (int8) {
    TrainArgs a;
    a.q = static_cast<const uint16_t*>(q);
    a.q8 = q8;
    a.k8 = k8;
    a.v8f = v8f;
    a.qs = qs;
    a.ks = ks;
    a.vs = vs;
    a.lut = lut;
    a.os = nullptr;
    a.os32 = os32;
    a.lse = lse;
    a.qphi = qphi;
    a.L = L;
    a.Nb = Nb;
    a.Np = Nb;
    a.Mb = Nb;
    a.T = T;
    a.n_tail = 0;
    a.Mq = Mq;
    a.qshift = qshift;
    a.Mqs = (int)((L + block_m - 1) / block_m);
    a.qsb = log2_exact(block_m);
    a.nwork = (int)nwork;
    a.per_xcd = (int)per_xcd;
    a.c2 = scale * 1.4426950408889634f;
    if (bf)
      sparse_fwd_qat_kernel<BF16><<<nblocks, 256, 0, st>>>(a);
    else
      sparse_fwd_qat_kernel<F16><<<nblocks, 256, 0, st>>>(a);
  } else {
    Fwd16Args a;
    a.q = static_cast<const uint16_t*>(q);
    a.k = static_cast<const uint16_t*>(k);
    a.vt = static_cast<const uint16_t*>(vt);
    a.lut = lut;
    a.os = nullptr;
    a.os32 = os32;
    a.lse = lse;
    a.qphi = qphi;
    a.L = L;
    a.Nb = Nb;
    a.Mq = Mq;
    a.qshift = qshift;
    a.T = T;
    a.nwork = (int)nwork;
    a.per_xcd = (int)per_xcd;
    a.c = scale * 1.4426950408889634f;
    if (bf)
      sparse_fwd16_kernel<BF16><<<nblocks, 256, 0, st>>>(a);
    else
      sparse_fwd16_kernel<F16><<<nblocks, 256, 0, st>>>(a);
  }
  const int err = (int)hipGetLastError();
  if (err != 0) return err;
  dim3 grid(Nb, B * H);
  auto Kp = static_cast<const uint16_t*>(k);
  auto Vp = static_cast<const uint16_t*>(v);
  auto O = static_cast<uint16_t*>(o);
  if (bf)
    linear_mix_score_kernel<BF16, true><<<grid, 256, 0, st>>>(qphi, Kp, Vp, Hall, zall, lut, T, Nb, os32, alpha, alpha_stride, L, Mq, qshift, H, eps_l, O, nullptr, nullptr);
  else
    linear_mix_score_kernel<F16, true><<<grid, 256, 0, st>>>(qphi, Kp, Vp, Hall, zall, lut, T, Nb, os32, alpha, alpha_stride, L, Mq, qshift, H, eps_l, O, nullptr, nullptr);
  return (int)hipGetLastError();
}

// Linear branch and mix of the 1-D SLA2 inference path (_lin_fwd3 through
// complement_linear_states, models/sla2_vendor/kernel_linear.py:446-513):
// comp holds the complement records of 16-bit block states
// (sla2h_hblocks_states + sla2h_complement over the plain LUT), qphi =
// softmax_D(Q) in the 16-bit type; o = alpha o_s + (1 - alpha) o_l.
extern "C" int sla2h_lin_fwd3(const void* qphi, const void* comp, const void* o_s,
                              const float* alpha, int alpha_stride, int dtype, int B, int H,
                              int64_t L, int D, int bq, float eps_l, void* o, void* stream) {
  SLA2H_CHECK_ARG(qphi && comp && o_s && alpha && o);
  SLA2H_CHECK_ARG(D == kT && (bq == 64 || bq == 128 || bq == 256) && alpha_stride >= 0);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && B * H <= 65535 && L > 0);
  const int Mb = (int)((L + kT - 1) / kT);
  const int Mq = (int)((L + bq - 1) / bq);
  const int qshift = log2_exact(bq / kT);
  dim3 grid(Mb, B * H);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto QP = static_cast<const uint16_t*>(qphi);
  auto C = static_cast<const unsigned char*>(comp);
  auto OS = static_cast<const uint16_t*>(o_s);
  auto O = static_cast<uint16_t*>(o);
  if (dtype == SLA2H_DTYPE_BF16)
    linear_mix_qat_kernel<BF16, true><<<grid, 256, 0, st>>>(QP, C, nullptr, OS, alpha, alpha_stride, L, Mq, qshift, H, eps_l, O, nullptr, nullptr);
  else
    linear_mix_qat_kernel<F16, true><<<grid, 256, 0, st>>>(QP, C, nullptr, OS, alpha, alpha_stride, L, Mq, qshift, H, eps_l, O, nullptr, nullptr);
  return (int)hipGetLastError();
}

extern "C" int sla2h_sparse_fwd_1d(const void* q, const void* k, const void* vt, const int32_t* lut,
                                   int dtype, int B, int H, int64_t L, int D, int bq, int bk,
                                   int T, float scale, void* o_s, float* lse, void* qphi,
                                   void* stream) {
  SLA2H_CHECK_ARG(q && k && vt && lut && o_s && lse && qphi);
  SLA2H_CHECK_ARG(D == kT && bk == kT && (bq == 64 || bq == 128 || bq == 256));
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && L > 0 && L * kT * 2 < (1ll << 31));
  const int Nb = (int)((L + kT - 1) / kT);
  SLA2H_CHECK_ARG(T >= 1 && T <= Nb && T <= kMaxJ);
  const int64_t nwork = (int64_t)Nb * B * H;
  const int64_t per_xcd = (nwork + 7) / 8;
  SLA2H_CHECK_ARG(8 * per_xcd < (1ll << 31));
  Fwd16Args a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.vt = static_cast<const uint16_t*>(vt);
  a.lut = lut;
  a.os = static_cast<uint16_t*>(o_s);
  a.lse = lse;
  a.qphi = static_cast<uint16_t*>(qphi);
  a.L = L;
  a.Nb = Nb;
  a.Mq = (int)((L + bq - 1) / bq);
  a.qshift = bq == 64 ? 0 : (bq == 128 ? 1 : 2);
  a.T = T;
  a.nwork = (int)nwork;
  a.per_xcd = (int)per_xcd;
  a.c = scale * 1.4426950408889634f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nblocks = (int)(8 * per_xcd);
  if (dtype == SLA2H_DTYPE_BF16)
    sparse_fwd16_kernel<BF16><<<nblocks, 256, 0, st>>>(a);
  else
    sparse_fwd16_kernel<F16><<<nblocks, 256, 0, st>>>(a);
  return (int)hipGetLastError();
}
