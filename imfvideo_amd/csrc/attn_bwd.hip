// Backward of the SLA2 cube attention's training forward through the
// straight-through estimator, gfx950 (_CubeQATFunction.backward,
// models/sla2_cube_qat.py:753-832):
//   sparse branch  re-differentiated in 16-bit from the UNQUANTISED q, k, v:
//                  p = exp2(min(q.k scale log2e - lse, 4)) with the INT8
//                  forward's lse, ds = p (do_s . v - delta), saturated at
//                  +-60000 and rounded to 16 bits before the dq / dk products,
//                  p rounded to 16 bits for dv (sla_kernel.py:117-184,
//                  models/sla2_cube_qat.py:986-1042);
//   linear branch  dqphi = g16 H16^T - s z^T per query block
//                  (kernel_linear.py:85-138), dh = complement sum of
//                  qphi^T g over the query blocks NOT routing a tile, then
//                  dkphi = v dh16^T + dz, dv_l = kphi dh16
//                  (models/sla2_cube_qat.py:1045-1104);
//   phi chains     dx = x_s + phi (dphi - <phi, dphi>), saturated
//                  (models/sla2_cube_qat.py:875-904).
//
// Kernels: bwd_prep (per 64-row block: gradient split, delta, g, s, the alpha
// segment sums and the per-block partial states P = qphi^T g and Pz =
// qphi^T s), then the dq kernel (per query block, key-split waves) and the
// dk/dv kernel (per key tile, waves split as query half x key half).  The complement GEMM of the
// partial states lives with the forward's complement (states.hip).
//
// The products that contract over a wave's rows (dq over 16 keys, dk and dv over 32
// queries) take those rows transposed as their A operand: the wave holds
// the rows row-major in LDS and reads the operand with the gfx950 transposing
// LDS read, so no transposed copy of q, k or do_s goes through memory.
#include "common.h"

#include <climits>

namespace sla2h {

namespace {

constexpr int kT = 64;
constexpr int kMaxJ = 1024;
constexpr int kRecH = 0, kRecZ = 32768, kRecBytes = 33280;
constexpr float kSat = 60000.f;

__device__ inline float sat(float x) { return fminf(fmaxf(x, -kSat), kSat); }

__device__ inline f32x4 mfma_f32_16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <typename T16>
__device__ inline float r16(float x) {
  return T16::to_f32(T16::from_f32(x));
}

template <typename T16>
__device__ inline u32x2 pack4(float a, float b, float c, float d) {
  return u32x2{pack_pair<T16>(a, b), pack_pair<T16>(c, d)};
}

// ---------------------------------------------------------------------------
// bwd_prep: one 64-row block b of one (b, h) per workgroup.
// ---------------------------------------------------------------------------
struct PrepArgs {
  const uint16_t* dout;
  const uint16_t* o_s;
  const uint16_t* o_l;
  const float* den;
  const uint16_t* qphi;
  const float* alpha;
  uint16_t* dos;
  float* delta;
  uint16_t* g16;
  float* s;
  float* seg;
  float* P;
  float* Pz;
  int64_t L;
  int Nb, H, alpha_stride;
  int Mq, qshift;  // alpha rows / seg: query blocks of 64 << qshift rows
};

template <typename T16>
__global__ __launch_bounds__(256) void bwd_prep_kernel(PrepArgs a) {
  __shared__ float qps[kT][kT + 1];  // qphi [row][d]
  __shared__ float gs[kT][kT + 1];   // saturated g [row][e]
  __shared__ float ss[kT];
  __shared__ float zp[4][kT];        // partial z sums of the four row quarters
  __shared__ float red[4];

  // thread: rows rb and rb + 32, channels c0 .. c0 + 7 (a wave's 16-byte
  // loads of one tensor cover 8 whole rows, 1 KB contiguous)
  const int blk = blockIdx.x, bh = blockIdx.y, h = bh % a.H;
  const int tid = threadIdx.x, rb = tid >> 3, c0 = (tid & 7) * 8;
  const float al = a.alpha[(int64_t)h * a.alpha_stride + (blk >> a.qshift)];

  uint4 u[2][4];  // [row half][dout, o_s, o_l, qphi]
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int64_t row = (int64_t)blk * kT + rb + 32 * hf;
    const int64_t off = ((int64_t)bh * a.L + row) * kT + c0;
    const bool valid = row < a.L;
    const uint16_t* src[4] = {a.dout, a.o_s, a.o_l, a.qphi};
#pragma unroll
    for (int t = 0; t < 4; ++t)
      u[hf][t] = valid ? *reinterpret_cast<const uint4*>(src[t] + off) : make_uint4(0, 0, 0, 0);
  }
  float segp = 0.f;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int r = rb + 32 * hf;
    const int64_t row = (int64_t)blk * kT + r;
    const bool valid = row < a.L;
    const int64_t off = ((int64_t)bh * a.L + row) * kT + c0;
    const float den = valid ? a.den[(int64_t)bh * a.L + row] : 1.f;
    const uint32_t wd[4][4] = {{u[hf][0].x, u[hf][0].y, u[hf][0].z, u[hf][0].w},
                               {u[hf][1].x, u[hf][1].y, u[hf][1].z, u[hf][1].w},
                               {u[hf][2].x, u[hf][2].y, u[hf][2].z, u[hf][2].w},
                               {u[hf][3].x, u[hf][3].y, u[hf][3].z, u[hf][3].w}};
    float dsum = 0.f, ssum = 0.f;
    uint32_t dso[4], g16o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint16_t dsb[2], gb[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const int sh = 16 * x;
        const float d = T16::to_f32((uint16_t)(wd[0][e] >> sh));
        const float os = T16::to_f32((uint16_t)(wd[1][e] >> sh));
        const float ol = T16::to_f32((uint16_t)(wd[2][e] >> sh));
        // (do * a).to(16-bit), (do * (1 - a)).to(16-bit) of the reference's
        // split kernel: the fp32 products round before the 16-bit conversion
        dsb[x] = T16::from_f32(d * al);
        const float dl = r16<T16>(d * (1.f - al));
        dsum += os * T16::to_f32(dsb[x]);
        segp += d * (os - ol);
        ssum += dl * ol;
        const float g = sat(dl / den);
        gs[r][c0 + 2 * e + x] = g;
        gb[x] = T16::from_f32(g);
        qps[r][c0 + 2 * e + x] = T16::to_f32((uint16_t)(wd[3][e] >> sh));
      }
      dso[e] = pack2(dsb[0], dsb[1]);
      g16o[e] = pack2(gb[0], gb[1]);
    }
#pragma unroll
    for (int m = 1; m <= 4; m <<= 1) {
      dsum += __shfl_xor(dsum, m, 64);
      ssum += __shfl_xor(ssum, m, 64);
    }
    const float srow = valid ? ssum / den : 0.f;
    if ((tid & 7) == 0) ss[r] = srow;
    if (valid) {
      *reinterpret_cast<uint4*>(a.dos + off) = make_uint4(dso[0], dso[1], dso[2], dso[3]);
      *reinterpret_cast<uint4*>(a.g16 + off) = make_uint4(g16o[0], g16o[1], g16o[2], g16o[3]);
      if ((tid & 7) == 0) {
        a.delta[(int64_t)bh * a.L + row] = dsum;
        a.s[(int64_t)bh * a.L + row] = srow;
      }
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) segp += __shfl_xor(segp, m, 64);
  if ((tid & 63) == 0) red[tid >> 6] = segp;
  __syncthreads();
  if (tid == 0)
    atomicAdd(a.seg + (int64_t)h * a.Mq + (blk >> a.qshift), (red[0] + red[1]) + (red[2] + red[3]));

  // P[d][e] = sum_rows qphi[row][d] g[row][e] on fp32 MFMA, computed as P^T so
  // that a lane holds four consecutive e of one d (16-byte stores): wave w owns
  // d 16w .. 16w + 15, lane (lg, lr) d = 16w + lr, e = 16et + 4lg .. + 3
  {
    const int w = tid >> 6, l = tid & 63, lr = l & 15, lg = l >> 4;
    f32x4 acc[4];
#pragma unroll
    for (int et = 0; et < 4; ++et) acc[et] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int kk = 0; kk < 16; ++kk) {
      const int rw = 4 * kk + lg;
      const float bv = qps[rw][16 * w + lr];
#pragma unroll
      for (int et = 0; et < 4; ++et) acc[et] = mfma_f32_16x16x4(gs[rw][16 * et + lr], bv, acc[et]);
    }
    float* P = a.P + ((int64_t)bh * a.Nb + blk) * (kT * kT) + (16 * w + lr) * kT + 4 * lg;
#pragma unroll
    for (int et = 0; et < 4; ++et) *reinterpret_cast<f32x4*>(P + 16 * et) = acc[et];
  }
  {  // z[d] = sum_rows qphi[row][d] s[row]: four row quarters, then their sum
    const int d = tid & 63, qr = tid >> 6;
    float z = 0.f;
#pragma unroll 4
    for (int rw = 16 * qr; rw < 16 * qr + 16; ++rw) z += qps[rw][d] * ss[rw];
    zp[qr][d] = z;
  }
  __syncthreads();
  if (tid < kT)
    a.Pz[((int64_t)bh * a.Nb + blk) * kT + tid] = (zp[0][tid] + zp[1][tid]) + (zp[2][tid] + zp[3][tid]);
}

// gfx950 transposing LDS read (ds_read_b64_tr_b16): within each group of 16
// lanes, lane j receives element j % 4 of the 8 bytes addressed by lanes
// j / 4, 4 + j / 4, 8 + j / 4 and 12 + j / 4 of its group, in that order.
__device__ inline u32x2 lds_read_tr16(const void* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
  return __builtin_bit_cast(u32x2, v);
}

// ---------------------------------------------------------------------------
// dq: one 64-row query block per workgroup; wave w owns keys 16w..16w+15 of
// every tile of the augmented LUT and all 64 queries.  Per tile and query
// group qb: S^T = K Q^T and dP^T = V do_s^T (16-bit MFMA, lane (g, r) holds
// keys 16w+4g+i of query 16qb+r), ds, then dq^T += K^T ds^T over the wave's 16
// keys.  The four key-split partials are summed through LDS, then wave w
// finishes queries 16w..16w+15: dq_s, the linear dqphi from the forward's
// complement record, and the phi chain.
// ---------------------------------------------------------------------------
struct DqArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* dos;
  const uint16_t* g16;
  const uint16_t* qphi;
  const float* lse;
  const float* delta;
  const float* s;
  const float* Hall;
  const unsigned char* comp;
  const int32_t* lut;
  uint16_t* dq;
  int64_t L;
  int Nb, J, nwork, per_xcd;
  int Mq, qshift;  // LUT rows and forward records per query block of 64 << qshift rows
  float c, scale;
};

template <typename T16>
__global__ __launch_bounds__(256, 2) void bwd_dq_kernel(DqArgs a) {
  __shared__ int tiles[kMaxJ];
  __shared__ __align__(16) f32x4 mb[2][4][2][4][64];  // [round-robin][src wave][qb sel][ct][lane]
  // 16-bit complement state H16[d][e] of this query block and its z, staged
  // while the prologue's other loads are in flight
  __shared__ __align__(16) uint16_t h16s[kT][kT + 8];
  __shared__ float zcs[kT];

  const int logical = (blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
  if (logical >= a.nwork) return;
  const int bh = __builtin_amdgcn_readfirstlane(logical / a.Nb);
  const int m = __builtin_amdgcn_readfirstlane(logical - bh * a.Nb);
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, r = l & 15, g = l >> 4;
  const int64_t L = a.L;
  const int64_t base = (int64_t)bh * L;

  const int mq = m >> a.qshift;
  const int32_t* lrow = a.lut + ((int64_t)bh * a.Mq + mq) * a.J;
  for (int j = tid; j < a.J; j += 256) {
    const int n = lrow[j];
    tiles[j] = n < 0 ? 0 : (n >= a.Nb ? a.Nb - 1 : n);
  }
  __syncthreads();
  // the augmented list in ascending tile order (dq sums over all of it)
  sort_ids_ascending(
      a.J, tid, [&](int i) { return tiles[i]; }, [&](int i, int v) { tiles[i] = v; },
      reinterpret_cast<int*>(&mb[0][0][0][0][0]));

  // resident B operands: Q and do_s rows 16qb + r, channels 32ks + 8g .. +7
  u32x4 qf[4][2], df[4][2];
  float lse_r[4], del_r[4];
#pragma unroll
  for (int qb = 0; qb < 4; ++qb) {
    const int64_t row = (int64_t)m * kT + 16 * qb + r;
    const bool ok = row < L;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      qf[qb][ks] = ok ? *reinterpret_cast<const u32x4*>(a.q + (base + row) * kT + 32 * ks + 8 * g)
                      : u32x4{0, 0, 0, 0};
      df[qb][ks] = ok ? *reinterpret_cast<const u32x4*>(a.dos + (base + row) * kT + 32 * ks + 8 * g)
                      : u32x4{0, 0, 0, 0};
    }
    lse_r[qb] = ok ? a.lse[base + row] : INFINITY;
    del_r[qb] = ok ? a.delta[base + row] : 0.f;
  }
  f32x4 ndel[4];  // -delta of each query group, the dP accumulators' start
#pragma unroll
  for (int qb = 0; qb < 4; ++qb) ndel[qb] = f32x4{-del_r[qb], -del_r[qb], -del_r[qb], -del_r[qb]};
  const unsigned char* rec = a.comp + ((int64_t)bh * a.Mq + mq) * kRecBytes;
  {  // H16 = round16(Hc + (round16(Hall) - Hall)); thread: row tid / 4, 16 columns
    const int d = tid >> 2, c0 = (tid & 3) * 16;
    const f32x4* hc = reinterpret_cast<const f32x4*>(rec + kRecH) + (d * kT + c0) / 4;
    const f32x4* ha = reinterpret_cast<const f32x4*>(a.Hall + (int64_t)bh * kT * kT) + (d * kT + c0) / 4;
    f32x4 hx[4], tx[4];
#pragma unroll
    for (int cq = 0; cq < 4; ++cq) {
      hx[cq] = hc[cq];
      tx[cq] = ha[cq];
    }
    uint32_t wd[8];
#pragma unroll
    for (int cq = 0; cq < 4; ++cq) {
      float hv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) hv[i] = hx[cq][i] + (r16<T16>(tx[cq][i]) - tx[cq][i]);
      wd[2 * cq] = pack_pair<T16>(hv[0], hv[1]);
      wd[2 * cq + 1] = pack_pair<T16>(hv[2], hv[3]);
    }
    *reinterpret_cast<uint4*>(&h16s[d][c0]) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    *reinterpret_cast<uint4*>(&h16s[d][c0 + 8]) = make_uint4(wd[4], wd[5], wd[6], wd[7]);
    if (tid < kT) zcs[tid] = reinterpret_cast<const float*>(rec + kRecZ)[tid];
  }
  __syncthreads();

  const auto rk = make_rsrc(a.k + base * kT, L * kT * 2);  // key rows past L read as 0
  const auto rv = make_rsrc(a.v + base * kT, L * kT * 2);
  // The wave's K and V rows of a tile (its 16 keys, 2 KB each) load as two
  // contiguous 1 KB halves (lane l: row 8 h + l / 8 of the 16, bytes
  // 16 (l % 8) ..): whole cache lines per load, where loading the MFMA
  // fragments directly (lane: one row, 16 bytes of each half-row) touches
  // twice the lines per instruction.  The rows go to the wave's own staging
  // slots in the merge buffer (free during the key loop: the sort is done,
  // the partial sums come after it), K in its first 8 KB and V in its second,
  // rows padded to 144 bytes against bank conflicts; the K and V fragments
  // and the transposed K^T operands are read back from there.
  constexpr int kKs = 144;
  const int rowoff = ((16 * w + (l >> 3)) * kT) * 2 + 16 * (l & 7);
  unsigned char* kst = reinterpret_cast<unsigned char*>(&mb[0][w][0][0][0]);
  unsigned char* vst = reinterpret_cast<unsigned char*>(&mb[1][w][0][0][0]);

  // score-side operands: the K and V rows of the wave's 16 keys as loaded
  // (the K rows also give the K^T operands of the dq product)
  struct Frags {
    u32x4 k[2], v[2];
  };
  auto load = [&](int j, Frags& f) {
    const int n = __builtin_amdgcn_readfirstlane(tiles[j]);
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // tile offset in voffset: range-checked, rows past L read 0
      f.k[h] = buf_load16(rk, n * kT * kT * 2 + rowoff + h * 8 * kT * 2, 0);
      f.v[h] = buf_load16(rv, n * kT * kT * 2 + rowoff + h * 8 * kT * 2, 0);
    }
  };
  auto stage = [&](const Frags& f, int slot) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int o = slot * 16 * kKs + (8 * h + (l >> 3)) * kKs + 16 * (l & 7);
      *reinterpret_cast<u32x4*>(kst + o) = f.k[h];
      *reinterpret_cast<u32x4*>(vst + o) = f.v[h];
    }
  };
  // MFMA fragments: lane (g, r) row r of the 16, channels 32 ks + 8 g .. + 7
  auto read_kv = [&](int slot, Frags& f) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int o = slot * 16 * kKs + r * kKs + 64 * ks + 16 * g;
      f.k[ks] = *reinterpret_cast<const u32x4*>(kst + o);
      f.v[ks] = *reinterpret_cast<const u32x4*>(vst + o);
    }
  };
  // K^T operand [channel 16 ct + r][key 16 w + 4 g + e]: this lane addresses
  // key row 4 g + r / 4, channels 16 ct + 4 (r % 4) .. + 3
  auto read_kt = [&](int slot, u32x2 (&kt)[4]) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
      kt[ct] = lds_read_tr16(kst + slot * 16 * kKs + (4 * g + (r >> 2)) * kKs + 2 * (16 * ct + 4 * (r & 3)));
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int qb = 0; qb < 4; ++qb)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[qb][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Keys past L need no mask here: their K and V rows read as zero (buffer
  // range check), so are their K^T operands, so dp = 0, ds stays
  // finite (p <= 2^4) and K^T ds adds exactly zero to dq.
  // ds^T fragments of one tile: lane (g, r) holds keys 16w+4g+i of query 16qb+r
  auto tile_ds = [&](const Frags& f, u32x2 (&dsp)[4]) {
#pragma unroll
    for (int qb = 0; qb < 4; ++qb) {
      f32x4 sc = mfma_16x16x32<T16>(f.k[0], qf[qb][0], f32x4{0.f, 0.f, 0.f, 0.f});
      sc = mfma_16x16x32<T16>(f.k[1], qf[qb][1], sc);
      // dP - delta straight from the matrix core: the accumulator starts at
      // -delta of the query (this lane's column), one VALU subtraction less
      // per score (the difference rounds once, as fl(dP - delta) does, but
      // the products are summed onto -delta)
      f32x4 dp = mfma_16x16x32<T16>(f.v[0], df[qb][0], ndel[qb]);
      dp = mfma_16x16x32<T16>(f.v[1], df[qb][1], dp);
      float ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = fast_exp2(fminf(sc[i] * a.c - lse_r[qb], 4.f));
        ds[i] = sat(p * dp[i]);
      }
      dsp[qb] = pack4<T16>(ds[0], ds[1], ds[2], ds[3]);
    }
  };
  // dq^T += K^T ds^T over the wave's 16 keys of one tile (K = 16), or of a pair
  // of tiles on one K = 32 product (operand slots 4..7 carry the second tile)
  auto dq_single = [&](const u32x2 (&kt)[4], const u32x2 (&dsp)[4]) {
#pragma unroll
    for (int qb = 0; qb < 4; ++qb)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) acc[qb][ct] = mfma_16x16x16<T16>(kt[ct], dsp[qb], acc[qb][ct]);
  };
  auto dq_pair = [&](const u32x2 (&kta)[4], const u32x2 (&dsa)[4], const u32x2 (&ktb)[4],
                     const u32x2 (&dsb)[4]) {
#pragma unroll
    for (int qb = 0; qb < 4; ++qb)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        acc[qb][ct] = mfma_16x16x32<T16>(u32x4{kta[ct].x, kta[ct].y, ktb[ct].x, ktb[ct].y},
                                         u32x4{dsa[qb].x, dsa[qb].y, dsb[qb].x, dsb[qb].y},
                                         acc[qb][ct]);
  };

  // Tiles in pairs: the second tile's rows are requested before the first
  // tile's scores, the next pair's first tile right after them.  Each tile's
  // rows go to the wave's staging slot once they arrive; its fragments, and
  // the K^T operands of the pair product, are read back from there.
  const int J = a.J;
  Frags fa, fb, op;
  u32x2 kta[4], ktb[4];
  load(0, fa);
  int j = 0;
  for (; j + 1 < J; j += 2) {
    u32x2 dsa[4], dsb[4];
    load(j + 1, fb);
    stage(fa, 0);
    read_kv(0, op);
    tile_ds(op, dsa);
    load(j + 2 < J ? j + 2 : J - 1, fa);
    stage(fb, 1);
    read_kv(1, op);
    tile_ds(op, dsb);
    read_kt(0, kta);
    read_kt(1, ktb);
    dq_pair(kta, dsa, ktb, dsb);
  }
  if (j < J) {
    u32x2 dsa[4];
    stage(fa, 0);
    read_kv(0, op);
    tile_ds(op, dsa);
    read_kt(0, kta);
    dq_single(kta, dsa);
  }

  // sum the key-split partials: round t moves query groups 2t, 2t+1
  f32x4 tot[4];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int qs = 0; qs < 2; ++qs)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) mb[t][w][qs][ct][l] = acc[2 * t + qs][ct];
  }
  __syncthreads();
  {
    const int t = w >> 1, qs = w & 1;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
      tot[ct] = (mb[t][0][qs][ct][l] + mb[t][1][qs][ct][l]) + (mb[t][2][qs][ct][l] + mb[t][3][qs][ct][l]);
  }

  // epilogue: query row 64m + 16w + r, channels 16ct + 4g + i
  const int64_t row = (int64_t)m * kT + 16 * w + r;
  const bool ok = row < L;
  u32x4 gb[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
    gb[ks] = ok ? *reinterpret_cast<const u32x4*>(a.g16 + (base + row) * kT + 32 * ks + 8 * g)
                : u32x4{0, 0, 0, 0};
  const float srow = ok ? a.s[base + row] : 0.f;
  float dqphi[4][4], qp[4][4];
  float dot = 0.f;
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    f32x4 num = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      // A: H16[d = 16ct + r][e = 32ks + 8g .. +7]
      const u32x4 av = *reinterpret_cast<const u32x4*>(&h16s[16 * ct + r][32 * ks + 8 * g]);
      num = mfma_16x16x32<T16>(av, gb[ks], num);
    }
    const f32x4 z = *reinterpret_cast<const f32x4*>(&zcs[16 * ct + 4 * g]);
    const uint2 qv = ok ? *reinterpret_cast<const uint2*>(a.qphi + (base + row) * kT + 16 * ct + 4 * g)
                        : make_uint2(0, 0);
    const uint32_t qw[2] = {qv.x, qv.y};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dqphi[ct][i] = num[i] - srow * z[i];
      qp[ct][i] = T16::to_f32((uint16_t)(qw[i >> 1] >> (16 * (i & 1))));
      dot += qp[ct][i] * dqphi[ct][i];
    }
  }
  dot = sum_over_groups(dot);
  if (ok) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float dqs = r16<T16>(tot[ct][i] * a.scale);
        o[i] = sat(dqs + qp[ct][i] * (dqphi[ct][i] - dot));
      }
      const u32x2 pk = pack4<T16>(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<u32x2*>(a.dq + (base + row) * kT + 16 * ct + 4 * g) = pk;
    }
  }
}

// ---------------------------------------------------------------------------
// dk, dv: one key tile per workgroup; wave w = 2 qh + kh owns queries
// 32qh..32qh+31 of each query block that routes the tile (ascending block
// order) and keys 32kh..32kh+31, whose K and V fragments it holds in
// registers.  Per block, key group kb and query sub-tile qt: S^T = Q K^T and
// dP = do_s V^T (lane (g, r) holds queries 32qh+16qt+4g+i of key
// 32kh+16kb+r), p and ds; then dv^T += do_s^T p and dk^T += Q^T ds over the
// wave's 32 queries on K = 32 products.  The two query-half partials are
// summed through LDS; wave w finishes keys 16w..16w+15: dk_s, dv_s, the
// linear dkphi / dv_l from the backward complement record, and the phi
// chain of K.
// ---------------------------------------------------------------------------
struct DkdvArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* dos;
  const float* lse;
  const float* delta;
  const uint32_t* sel;
  const unsigned char* compb;
  uint16_t* dk;
  uint16_t* dv;
  int64_t L;
  int Nb, NCq, nwork, per_xcd;
  float c, scale;
};

// Prefetch region of one wave: 4 slots of 64 lanes x 16 B, then lse and delta
// (64 dwords each).  The four regions also hold the partial-sum exchange
// after the loop (32 KB).
constexpr int kPfSlot = 1024;
constexpr int kPfWave = 8 * kPfSlot + 2 * 256;
constexpr int kPoolBytes = 4 * kPfWave > 32768 ? 4 * kPfWave : 32768;
constexpr int kSelLds = 128;  // mask words staged in LDS (query blocks 0 .. 4095)
// s_waitcnt immediates (gfx9 encoding): vmcnt(0) alone, lgkmcnt(0) alone
constexpr int kWaitVm0 = 0x0F70;
constexpr int kWaitLgkm0 = 0xC07F;

// Buffer loads straight into LDS: lane l's bytes land at dst + l * size.
// dst must be wave-uniform; offsets past the resource's range write zeros.
__device__ inline void lds_load16(__amdgpu_buffer_rsrc_t rs, void* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)dst, 16,
                                           voff, 0, 0, 0);
}
__device__ inline void lds_load4(__amdgpu_buffer_rsrc_t rs, void* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)dst, 4,
                                           voff, 0, 0, 0);
}

template <typename T16>
__global__ __launch_bounds__(256, 2) void bwd_dkdv_kernel(DkdvArgs a) {
  __shared__ __align__(16) uint16_t kv[2][kT][kT + 8];   // K, V rows of the tile
  __shared__ __align__(16) uint16_t dhs[2][kT][kT + 8];  // dh16 [d][e], dh16^T [e][d]
  // Per-wave prefetch regions of the query-block loop; after the loop the
  // same bytes hold the partial-sum exchange mb[src wave][kb sel][ct][lane].
  __shared__ __align__(16) unsigned char pool[kPoolBytes];
  __shared__ float dzs[kT];
  __shared__ uint32_t selsh[kSelLds];  // first words of this tile's query-block mask
  auto mb = reinterpret_cast<f32x4 (*)[2][4][64]>(pool);

  const int logical = (blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
  if (logical >= a.nwork) return;
  const int bh = __builtin_amdgcn_readfirstlane(logical / a.Nb);
  const int n = __builtin_amdgcn_readfirstlane(logical - bh * a.Nb);
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63, r = l & 15, g = l >> 4;
  const int64_t L = a.L;
  const int64_t base = (int64_t)bh * L;

  {  // stage K, V rows (zero past L) and the complement state dh (saturated, 16-bit)
    const int rr = tid >> 2, c0 = (tid & 3) * 16;
    const int64_t row = (int64_t)n * kT + rr;
    const bool ok = row < L;
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const uint16_t* src = (x == 0 ? a.k : a.v) + (base + row) * kT + c0;
      uint4 u0 = make_uint4(0, 0, 0, 0), u1 = u0;
      if (ok) {
        u0 = reinterpret_cast<const uint4*>(src)[0];
        u1 = reinterpret_cast<const uint4*>(src)[1];
      }
      *reinterpret_cast<uint4*>(&kv[x][rr][c0]) = u0;
      *reinterpret_cast<uint4*>(&kv[x][rr][c0 + 8]) = u1;
    }
    const unsigned char* rec = a.compb + ((int64_t)bh * a.Nb + n) * kRecBytes;
    const f32x4* hr = reinterpret_cast<const f32x4*>(rec + kRecH) + (rr * kT + c0) / 4;
#pragma unroll
    for (int cq = 0; cq < 4; ++cq) {
      const f32x4 x = hr[cq];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint16_t hb = T16::from_f32(sat(x[i]));
        dhs[0][rr][c0 + 4 * cq + i] = hb;
        dhs[1][c0 + 4 * cq + i][rr] = hb;
      }
    }
    if (tid < kT) dzs[tid] = -reinterpret_cast<const float*>(rec + kRecZ)[tid];
  }
  const uint32_t* selrow = a.sel + ((int64_t)bh * a.Nb + n) * a.NCq;
  for (int j = tid; j < a.NCq && j < kSelLds; j += 256) selsh[j] = selrow[j];
  __syncthreads();

  // Wave w = 2 qh + kh takes query half qh (rows 32 qh .. + 31 of each routed
  // block, two 16-row sub-tiles qt) and key half kh (keys 32 kh .. + 31, two
  // 16-key groups kb'): 16 scores per lane per block, and the dk / dv products
  // contract over the wave's 32 queries on K = 32 MFMAs (32 MFMAs per wave and
  // block).  The two partials of a key half are summed after the loop.
  const int qh = w >> 1, kh = w & 1;
  f32x4 dkT[4][2], dvT[4][2];  // [ct][kb'] for keys 32 kh + 16 kb' + r
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) dkT[ct][kb] = dvT[ct][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 kres[2][2], vres[2][2];  // K, V fragments of the wave's keys, held for the whole loop
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      kres[kb][ks] = *reinterpret_cast<const u32x4*>(&kv[0][32 * kh + 16 * kb + r][32 * ks + 8 * g]);
      vres[kb][ks] = *reinterpret_cast<const u32x4*>(&kv[1][32 * kh + 16 * kb + r][32 * ks + 8 * g]);
    }

  // Query blocks m routed to this tile, ascending.  The operands of block m
  // (this wave's 32 query rows) are fetched one block ahead straight into the
  // wave's LDS region (buffer loads to LDS: no registers held in flight):
  // eight slots of 64 lanes x 16 B -- Q rows 0-7, 8-15, 16-23, 24-31, then the
  // do_s rows alike, each slot one contiguous 1 KB of the row-major tensor,
  // lane l fetching row l / 8, 16-byte chunk (l % 8) ^ (l / 8) (the XOR
  // spreads the 16 rows read by one fragment load over all banks) -- then 64
  // dwords of lse and 64 of delta (query 32 qh + (lane & 31)).  The two waves
  // of a query half fetch the same rows, each into its own region, so no wave
  // waits on another inside the loop.  Rows past L read as zero: such a query
  // then has p = 1 but zero Q and do_s rows, so it adds exactly zero to dk and
  // dv (as with a masked p).
  const auto rq = make_rsrc(a.q + base * kT, L * kT * 2);
  const auto rdo = make_rsrc(a.dos + base * kT, L * kT * 2);
  const auto rls = make_rsrc(a.lse + base, L * 4);
  const auto rdl = make_rsrc(a.delta + base, L * 4);
  unsigned char* pf = pool + w * kPfWave;
  auto prefetch = [&](int m) {
    const int rowb = (m * kT + 32 * qh + (l >> 3)) * (kT * 2) + 16 * ((l & 7) ^ (l >> 3));
    const int qo = (m * kT + 32 * qh + (l & 31)) * 4;
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) lds_load16(rq, pf + sl * kPfSlot, rowb + sl * 8 * kT * 2);
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) lds_load16(rdo, pf + (4 + sl) * kPfSlot, rowb + sl * 8 * kT * 2);
    lds_load4(rls, pf + 8 * kPfSlot, qo);
    lds_load4(rdl, pf + 8 * kPfSlot + 256, qo);
  };
  int kc = 0;
  uint32_t bits = 0u;
  if (a.NCq > 0) bits = __builtin_amdgcn_readfirstlane(selsh[0]);
  auto next_block = [&]() -> int {
    while (bits == 0u) {
      if (++kc >= a.NCq) return -1;
      bits = __builtin_amdgcn_readfirstlane(kc < kSelLds ? selsh[kc] : selrow[kc]);
    }
    const int m = 32 * kc + __builtin_ctz(bits);
    bits &= bits - 1u;
    return m;
  };

  int m = next_block();
  if (m >= 0) prefetch(m);
  while (m >= 0) {
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // this wave's prefetch of block m has landed
    u32x4 qa[2][2], da[2][2];  // [qt][ks]
    u32x4 qT[4], dT[4];        // [ct]: queries of sub-tile 0 in .xy, of sub-tile 1 in .zw
    float lse4[2][4], del4[2][4];
    {
      // Q, do_s A operands: lane (g, r) takes row 16 qt + r, chunk 4 ks + g
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int rho = 16 * qt + r;
          const int off = (rho >> 3) * kPfSlot + ((rho & 7) * 8 + ((4 * ks + g) ^ (rho & 7))) * 16;
          qa[qt][ks] = *reinterpret_cast<const u32x4*>(pf + off);
          da[qt][ks] = *reinterpret_cast<const u32x4*>(pf + 4 * kPfSlot + off);
        }
      // Q^T, do_s^T operands [channel 16 ct + r][query 16 qt + 4 g + e], read
      // transposed from the rows: this lane addresses row rho = 16 qt + 4 g +
      // r / 4, channels 16 ct + 4 (r % 4) .. + 3, i.e. chunk 2 ct + (r % 4) / 2
      // of that row at byte 8 (r % 2), placed by the prefetch as above
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        u32x2 t[2][2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          const int rho = 16 * qt + 4 * g + (r >> 2);
          const int off = (rho >> 3) * kPfSlot +
                          ((rho & 7) * 8 + ((2 * ct + ((r & 3) >> 1)) ^ (rho & 7))) * 16 + 8 * (r & 1);
          t[0][qt] = lds_read_tr16(pf + off);
          t[1][qt] = lds_read_tr16(pf + 4 * kPfSlot + off);
        }
        qT[ct] = u32x4{t[0][0].x, t[0][0].y, t[0][1].x, t[0][1].y};
        dT[ct] = u32x4{t[1][0].x, t[1][0].y, t[1][1].x, t[1][1].y};
      }
      // lse, delta of queries 32 qh + 16 qt + 4 g + i
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const f32x4 ls = *reinterpret_cast<const f32x4*>(pf + 8 * kPfSlot + 64 * qt + 16 * g);
        const f32x4 dl = *reinterpret_cast<const f32x4*>(pf + 8 * kPfSlot + 256 + 64 * qt + 16 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lse4[qt][i] = ls[i];
          del4[qt][i] = dl[i];
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // the region is read: free for the next block
    const int mn = next_block();
    if (mn >= 0) prefetch(mn);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      u32x2 pp[2], dsp[2];
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        // dP - delta from the matrix core (accumulator started at -delta of
        // the query rows 16 qt + 4g + i this lane holds)
        f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
        f32x4 dp = f32x4{-del4[qt][0], -del4[qt][1], -del4[qt][2], -del4[qt][3]};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          sc = mfma_16x16x32<T16>(qa[qt][ks], kres[kb][ks], sc);
          dp = mfma_16x16x32<T16>(da[qt][ks], vres[kb][ks], dp);
        }
        // p and ds of a (query, key) pair feed only that key's dk / dv column.
        // A key past L (zero K row) needs no mask and its p no clamp: whatever
        // its p, its column is never stored.  A query past L has zero Q and
        // do_s rows and lse 0, so p = 1 and it adds exactly zero.
        float p[4], ds[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = fast_exp2(sc[i] * a.c - lse4[qt][i]);
          ds[i] = sat(p[i] * dp[i]);
        }
        pp[qt] = pack4<T16>(p[0], p[1], p[2], p[3]);
        dsp[qt] = pack4<T16>(ds[0], ds[1], ds[2], ds[3]);
      }
      // K = 32 over the wave's queries: k index 8 g + j is query 16 (j / 4) +
      // 4 g + j % 4 in both operands
      const u32x4 pb = u32x4{pp[0].x, pp[0].y, pp[1].x, pp[1].y};
      const u32x4 db = u32x4{dsp[0].x, dsp[0].y, dsp[1].x, dsp[1].y};
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        dvT[ct][kb] = mfma_16x16x32<T16>(dT[ct], pb, dvT[ct][kb]);
        dkT[ct][kb] = mfma_16x16x32<T16>(qT[ct], db, dkT[ct][kb]);
      }
    }
    m = mn;
  }

  // sum the two query-half partials of each key half: wave w keeps key group
  // 16 w .. 16 w + 15 = key half w / 2, group w % 2, from waves w / 2 and 2 + w / 2
  f32x4 dkt[4], dvt[4];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    __syncthreads();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) mb[w][kb][ct][l] = x == 0 ? dkT[ct][kb] : dvT[ct][kb];
    __syncthreads();
    const int sh = w >> 1, sk = w & 1;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const f32x4 sum = mb[sh][sk][ct][l] + mb[2 + sh][sk][ct][l];
      if (x == 0)
        dkt[ct] = sum;
      else
        dvt[ct] = sum;
    }
  }

  // epilogue: key row 64n + 16w + r, channels 16ct + 4g + i
  const int kr = 16 * w + r;
  // phi(K) row statistics from this lane's channels 32ks + 8g .. +7
  float kx[2][8];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const u32x4 u = *reinterpret_cast<const u32x4*>(&kv[0][kr][32 * ks + 8 * g]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      kx[ks][2 * e] = T16::to_f32((uint16_t)(u[e] & 0xffff));
      kx[ks][2 * e + 1] = T16::to_f32((uint16_t)(u[e] >> 16));
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, kx[ks][e]);
  mx = max_over_groups(mx);
  float den = 0.f;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      kx[ks][e] = __expf(kx[ks][e] - mx);
      den += kx[ks][e];
    }
  den = sum_over_groups(den);
  u32x4 kpb[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int e = 0; e < 4; ++e) kpb[ks][e] = pack_pair<T16>(kx[ks][2 * e] / den, kx[ks][2 * e + 1] / den);

  float dkphi[4][4], dvl[4][4], kp[4][4];
  float dot = 0.f;
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    f32x4 x1 = f32x4{0.f, 0.f, 0.f, 0.f}, x2 = x1;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const u32x4 vb = *reinterpret_cast<const u32x4*>(&kv[1][kr][32 * ks + 8 * g]);
      const u32x4 ha = *reinterpret_cast<const u32x4*>(&dhs[0][16 * ct + r][32 * ks + 8 * g]);
      const u32x4 hta = *reinterpret_cast<const u32x4*>(&dhs[1][16 * ct + r][32 * ks + 8 * g]);
      x1 = mfma_16x16x32<T16>(ha, vb, x1);    // dkphi^T[d][key] = sum_e dh[d][e] V[key][e]
      x2 = mfma_16x16x32<T16>(hta, kpb[ks], x2);  // dv_l^T[e][key] = sum_d dh[d][e] kphi[key][d]
    }
    const uint2 kvv = *reinterpret_cast<const uint2*>(&kv[0][kr][16 * ct + 4 * g]);
    const uint32_t kw[2] = {kvv.x, kvv.y};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dkphi[ct][i] = x1[i] + dzs[16 * ct + 4 * g + i];
      dvl[ct][i] = x2[i];
      const float kxv = T16::to_f32((uint16_t)(kw[i >> 1] >> (16 * (i & 1))));
      kp[ct][i] = r16<T16>(__expf(kxv - mx) / den);
      dot += kp[ct][i] * dkphi[ct][i];
    }
  }
  dot = sum_over_groups(dot);
  const int64_t row = (int64_t)n * kT + kr;
  if (row < L) {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      float ok_[4], ov[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float dks = r16<T16>(dkt[ct][i] * a.scale);
        ok_[i] = sat(dks + kp[ct][i] * (dkphi[ct][i] - dot));
        ov[i] = sat(r16<T16>(dvt[ct][i]) + dvl[ct][i]);
      }
      *reinterpret_cast<u32x2*>(a.dk + (base + row) * kT + 16 * ct + 4 * g) = pack4<T16>(ok_[0], ok_[1], ok_[2], ok_[3]);
      *reinterpret_cast<u32x2*>(a.dv + (base + row) * kT + 16 * ct + 4 * g) = pack4<T16>(ov[0], ov[1], ov[2], ov[3]);
    }
  }
}

}  // namespace

}  // namespace sla2h

using namespace sla2h;

extern "C" int sla2h_bwd_prep(const void* dout, const void* o_s, const void* o_l, const float* den,
                              const void* qphi, const float* alpha, int alpha_stride, int dtype,
                              int B, int H, int64_t L, int D, int E, void* dos, float* delta,
                              void* g16, float* s, float* seg, float* P, float* Pz, void* stream) {
  SLA2H_CHECK_ARG(dout && o_s && o_l && den && qphi && alpha && dos && delta && g16 && s && seg &&
                  P && Pz);
  SLA2H_CHECK_ARG(D == kT && (E == 64 || E == 128 || E == 256) && alpha_stride >= 0);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && B * H <= 65535 && L > 0);
  PrepArgs a;
  a.qshift = E == 64 ? 0 : (E == 128 ? 1 : 2);
  a.Mq = (int)((L + E - 1) / E);
  a.dout = static_cast<const uint16_t*>(dout);
  a.o_s = static_cast<const uint16_t*>(o_s);
  a.o_l = static_cast<const uint16_t*>(o_l);
  a.den = den;
  a.qphi = static_cast<const uint16_t*>(qphi);
  a.alpha = alpha;
  a.dos = static_cast<uint16_t*>(dos);
  a.delta = delta;
  a.g16 = static_cast<uint16_t*>(g16);
  a.s = s;
  a.seg = seg;
  a.P = P;
  a.Pz = Pz;
  a.L = L;
  a.Nb = (int)((L + kT - 1) / kT);
  a.H = H;
  a.alpha_stride = alpha_stride;
  dim3 grid(a.Nb, B * H);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SLA2H_DTYPE_BF16)
    bwd_prep_kernel<BF16><<<grid, 256, 0, st>>>(a);
  else
    bwd_prep_kernel<F16><<<grid, 256, 0, st>>>(a);
  return (int)hipGetLastError();
}

extern "C" int sla2h_bwd_dq(const void* q, const void* k, const void* v, const void* dos,
                            const float* lse, const float* delta, const void* g16, const float* s,
                            const void* comp, const float* Hall, const void* qphi,
                            const int32_t* lut_aug, int dtype, int B, int H, int64_t L, int D,
                            int E, int J, float scale, void* dq, void* stream) {
  SLA2H_CHECK_ARG(q && k && v && dos && lse && delta && g16 && s && comp && Hall && qphi &&
                  lut_aug && dq);
  SLA2H_CHECK_ARG(D == kT && (E == 64 || E == 128 || E == 256) && scale > 0.f);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && L > 0 && J >= 1 && J <= kMaxJ);
  const int Nb = (int)((L + kT - 1) / kT);
  const int64_t nwork = (int64_t)Nb * B * H;
  const int64_t per_xcd = (nwork + 7) / 8;
  SLA2H_CHECK_ARG(8 * per_xcd < (1ll << 31) && L * kT * 2 < (1ll << 31));
  DqArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.dos = static_cast<const uint16_t*>(dos);
  a.g16 = static_cast<const uint16_t*>(g16);
  a.qphi = static_cast<const uint16_t*>(qphi);
  a.lse = lse;
  a.delta = delta;
  a.s = s;
  a.Hall = Hall;
  a.comp = static_cast<const unsigned char*>(comp);
  a.lut = lut_aug;
  a.dq = static_cast<uint16_t*>(dq);
  a.L = L;
  a.Nb = Nb;
  a.J = J;
  a.qshift = E == 64 ? 0 : (E == 128 ? 1 : 2);
  a.Mq = (int)((L + E - 1) / E);
  a.nwork = (int)nwork;
  a.per_xcd = (int)per_xcd;
  a.c = scale * 1.4426950408889634f;
  a.scale = scale;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nblocks = (int)(8 * per_xcd);
  if (dtype == SLA2H_DTYPE_BF16)
    bwd_dq_kernel<BF16><<<nblocks, 256, 0, st>>>(a);
  else
    bwd_dq_kernel<F16><<<nblocks, 256, 0, st>>>(a);
  return (int)hipGetLastError();
}

extern "C" int sla2h_bwd_dkdv(const void* q, const void* k, const void* v, const void* dos,
                              const float* lse, const float* delta, const uint32_t* sel,
                              const void* comp_bwd, int dtype, int B, int H, int64_t L, int D,
                              int E, float scale, void* dk, void* dv, void* stream) {
  SLA2H_CHECK_ARG(q && k && v && dos && lse && delta && sel && comp_bwd && dk && dv);
  SLA2H_CHECK_ARG(D == kT && E == kT && scale > 0.f);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && L > 0);
  const int Nb = (int)((L + E - 1) / E);
  const int64_t nwork = (int64_t)Nb * B * H;
  const int64_t per_xcd = (nwork + 7) / 8;
  SLA2H_CHECK_ARG(8 * per_xcd < (1ll << 31));
  DkdvArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.dos = static_cast<const uint16_t*>(dos);
  a.lse = lse;
  a.delta = delta;
  a.sel = sel;
  a.compb = static_cast<const unsigned char*>(comp_bwd);
  a.dk = static_cast<uint16_t*>(dk);
  a.dv = static_cast<uint16_t*>(dv);
  a.L = L;
  a.Nb = Nb;
  a.NCq = (Nb + 31) / 32;
  a.nwork = (int)nwork;
  a.per_xcd = (int)per_xcd;
  a.c = scale * 1.4426950408889634f;
  a.scale = scale;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nblocks = (int)(8 * per_xcd);
  if (dtype == SLA2H_DTYPE_BF16)
    bwd_dkdv_kernel<BF16><<<nblocks, 256, 0, st>>>(a);
  else
    bwd_dkdv_kernel<F16><<<nblocks, 256, 0, st>>>(a);
  return (int)hipGetLastError();
}
