// Fused SLA2 sparse + linear attention with forward-mode JVP, gfx950.
//
// Work unit: one 64-row query block m of one (b, h), one workgroup of 4
// wave64, over the block's key tiles (T routed video tiles + n_tail prefix
// blocks).  Primal only, wave w takes all 64 queries (four 16-row sub-tiles)
// and keys 16w..16w+15 of every tile; the four partial softmax states are
// merged once at the end through LDS.  With the tangent (twice the
// accumulators) wave w takes the query half w >> 1 (two sub-tiles) and the
// key half w & 1 of every tile, whose two 16-key quarters share the K = 32
// products of O; the two waves of a query half merge their states at the end.
// Either way each key tile is fetched once per query block, and each wave
// streams its part of every key tile straight from global memory into MFMA
// operand registers (one step ahead) -- no barriers in the key loop.  One
// pass over the tiles with a lazy running maximum: it moves only when a tile
// exceeds it by a margin (one wave ballot per tile), so the accumulators are
// rescaled about once per row.
//
// Scores are computed transposed (S^T = K Q^T) so that a lane holds one query
// column: the S^T fragment is directly the B operand of O^T = V^T P^T, and the
// per-query statistics stay lane-resident.
//
// Workgroup ids are remapped so that each XCD (ids = x mod 8) processes a
// contiguous range of work units: the query blocks of one head land on the
// same XCD and share its L2.
//
// Reference semantics: models/sla2_cube_qat.py:448-602 (_cube_fused_jvp_kernel),
// sparse-only variant :59-169 (_sla2_cube_jvp_qat_kernel).
#include "common.h"

#include <atomic>
#include <climits>
#include <type_traits>

namespace sla2h {

constexpr int kTa = 64;
constexpr size_t kRec = 2 * 16384 + 2 * 256;
constexpr int kMaxTiles = 1024;  // T + n_tail per query block

struct FwdArgs {
  const uint16_t* q;
  const uint16_t* dq;
  const uint16_t* kt;   // key-operand tiles [K|dK] in fragment order (tangent only)
  const uint16_t* vt;   // value-operand tiles (V, or V|dV with tangent) in fragment order
  const int8_t* q8;
  const int8_t* k8;
  const float* qs;
  const float* ks;
  const unsigned char* comp;
  const float* alpha;
  const int32_t* lut;
  const float* kb;     // per key tile: bound on ||k8_j|| ks over its rows (quant_pool), or null
  float* o;
  float* dout;
  int64_t L;
  int H, Nb, Np, Mb, T, n_tail, alpha_stride, nwork, per_xcd;
  int prescale;  // scale is a power of two (folded exactly into bf16 Q-side operands)
  int qshift;    // LUT rows, alpha and records per query block of 64 << qshift rows
  int Mq;        // LUT rows per (b, h)
  int ragged;    // id of a partial key tile that routed lists may hold, or -1
  float scale, c_log2, eps_l;
  float c16;     // log2-domain factor of the 16-bit primal scores
};

// bf16 x 2^k, exact for a power-of-two scale (no bf16 subnormals in range)
__device__ inline u32x4 scale_bf16x8(u32x4 u, float s) {
  u32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = bf16_val((uint16_t)(u[e] & 0xffff)) * s;
    const float hi = bf16_val((uint16_t)(u[e] >> 16)) * s;
    r[e] = pack2(bf16_bits(lo), bf16_bits(hi));
  }
  return r;
}

// A-operand fragment of H^T for numerator MFMAs: 8 consecutive d = 32 ks + 8 g + j
// of a record's fp32 H[d][v] at one column v, split into bf16 hi/lo halves.
__device__ inline void split_hfrag(const float (&x)[8], u32x4& hi, u32x4& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t h = pack_pair<BF16>(x[2 * e], x[2 * e + 1]);
    hi[e] = h;
    lo[e] = pack_pair<BF16>(x[2 * e] - bf16_val((uint16_t)(h & 0xffff)),
                            x[2 * e + 1] - bf16_val((uint16_t)(h >> 16)));
  }
}

struct KeyRegs {   // score-side operands, loaded one tile ahead
  i32x4 k8;      // K8[key 16w + r][16g .. 16g+15]
  u32x4 ka[4];   // ks 0,1: K[key][32ks + 8g ..], ks 2,3: dK[key][32(ks-2) + 8g ..]
};
struct ValRegs {   // value-side operands, loaded at the start of their own tile
  // per column tile ct: V[keys 16w + 4g .. +3][c = 16ct + r] in .xy and, with
  // tangent, dV of the same keys in .zw (one 16-byte load)
  u32x4 v[4];
};

// S16: primal scores from the 16-bit K Q^T (the K half of the kt operands and
// the Q half of the [dQ|Q] operands) instead of INT8 (the 1-D SLA2 JVP).
// Two workgroups per CU with the tangent (its registers), three primal only.
template <typename T16, bool TAN, bool LINEAR, bool PRE, bool S16>
__global__ __launch_bounds__(256, TAN ? 2 : 3) void fwd_jvp_kernel(FwdArgs a) {
  constexpr int kQT = TAN ? 2 : 4;  // 16-row query sub-tiles per wave
  __shared__ float stat[3][4][kQT][16];  // [m,l,mu][wave][qt][r]
  // [dQ|Q] B-operand fragments [sub-tile][ks][lane] (16 B each, tangent only)
  __shared__ __align__(16) u32x4 qsh[TAN ? 4 : 1][4][64];
  __shared__ __align__(16) i32x4 q8sh[4][64];  // INT8 Q B-operand fragments per sub-tile
  // cross-wave merge buffer [wave][slot][lane][4], 8 KB per wave: primal the
  // two column tiles of a round for the four sub-tiles (slot 4 cc + qt); with
  // the tangent O and dO of the four column tiles of one sub-tile (2 ct + {0,1})
  __shared__ __align__(16) float mbuf[4][8][64][4];
  // key tiles of this query block in visiting order: (tile id, key scale)
  __shared__ int2 tiles[kMaxTiles];
  __shared__ int ragged_last;  // the partial key tile was moved to the end of the routed list
  __shared__ float wmax[2][4];  // per wave: max kb, max ks over the block's key tiles
  __shared__ int redo;          // a row of the static-shift pass came out below its range

  // With the tangent the workgroups are persistent: slot s of XCD x takes the
  // XCD's units s, s + slots, ... in turn (the dispatch order of the one-shot
  // grid), so one unit's output stores and the next unit's operand loads
  // overlap instead of every workgroup of a round issuing them at once.
  // Primal only, one unit per workgroup (the loop body runs once; its
  // registers leave no room for the loop).
  const int slots = (int)(gridDim.x >> 3);
  for (int kk = (int)(blockIdx.x >> 3); kk < a.per_xcd; kk += slots) {
    const int logical = (blockIdx.x & 7) * a.per_xcd + kk;
    if (logical >= a.nwork) break;  // uniform: the whole workgroup leaves
    __syncthreads();  // the previous unit's LDS is free
    // integer division runs on the VALU: pin the (uniform) results to SGPRs so
    // that every pointer and buffer descriptor derived from them stays scalar
    const int bh = __builtin_amdgcn_readfirstlane(logical / a.Mb);
    const int m = __builtin_amdgcn_readfirstlane(logical - bh * a.Mb);
    const int h = __builtin_amdgcn_readfirstlane(bh % a.H);

    const int tid = threadIdx.x;
    // wave index uniform (SGPR) and lane index from mbcnt: neither holds a
    // VGPR across the key loop
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l = __lane_id(), r = l & 15, g = l >> 4;
    const int qs0 = TAN ? 2 * (w >> 1) : 0;  // first query sub-tile of the wave
    const int kq0 = TAN ? 2 * (w & 1) : w;   // first 16-key quarter of the wave
    const int64_t L = a.L;
    const int64_t qkbase = (int64_t)bh * L;
    const int64_t q0 = (int64_t)m * kTa;  // first query row of the block
    // element offset of the block's first row (uniform); per-lane offsets
    // within the block stay 32-bit, so no 64-bit lane address lives across the
    // key loop
    const int64_t blk = (qkbase + q0) * kTa;

    // ---- query side: INT8 and 16-bit [dQ|Q] B operands staged once in LDS,
    // wave w loading sub-tile w.
    {
      const int64_t row = q0 + 16 * w + r;
      const bool ok = row < L;
      const int ro = (16 * w + r) * kTa;
      if (!S16)
        q8sh[w][l] = ok ? *reinterpret_cast<const i32x4*>(a.q8 + blk + ro + 16 * g)
                        : i32x4{0, 0, 0, 0};
      if (TAN) {
#pragma unroll
        for (int part = 0; part < 2; ++part) {  // dQ in ks 0,1, Q in ks 2,3
          const uint16_t* src = part ? a.q : a.dq;
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            u32x4 v = ok ? *reinterpret_cast<const u32x4*>(src + blk + ro + 32 * ks + 8 * g)
                         : u32x4{0, 0, 0, 0};
            if (PRE) v = scale_bf16x8(v, a.scale);
            qsh[w][ks + 2 * part][l] = v;
          }
        }
      }
    }
    const int mq = m >> a.qshift;  // LUT row, alpha and record of this query block
    const int32_t* lrow = a.lut + ((int64_t)bh * a.Mq + mq) * a.T;
    const int J = a.T + a.n_tail;
    for (int j = tid; j < J; j += 256) {
      int n = j < a.T ? lrow[j] : a.Np + (j - a.T);
      n = n < 0 ? 0 : (n >= a.Nb ? a.Nb - 1 : n);  // out-of-range ids are clamped
      tiles[j].x = n;
    }
    __syncthreads();
    // routed tiles in ascending id order (the prefix tails stay at the end)
    sort_ids_ascending(
        a.T, tid, [&](int i) { return tiles[i].x; }, [&](int i, int v) { tiles[i].x = v; },
        reinterpret_cast<int*>(&mbuf[0][0][0][0]));
    // A partial key tile (1-D blocks over a ragged L) can sit anywhere in a routed
    // list: move it to the end, where the masked one-tile path handles it.
    int Tu = a.T;
    if (a.ragged >= 0) {
      if (tid == 0) {
        int found = 0;
        for (int j = 0; j < a.T; ++j) {
          if (tiles[j].x == a.ragged) {
            const int2 t = tiles[j];
            tiles[j] = tiles[a.T - 1];
            tiles[a.T - 1] = t;
            found = 1;
            break;
          }
        }
        ragged_last = found;
      }
      __syncthreads();
      Tu = a.T - ragged_last;
    }
    // key scales of the tiles in visiting order; the barrier that publishes
    // them comes after the first key loads are issued (their latencies overlap)
    if (!S16) {
      float kbm = 0.f, ksm = 0.f;
      for (int j = tid; j < J; j += 256) {
        const int64_t ti = (int64_t)bh * a.Nb + tiles[j].x;
        const float ksj = a.ks[ti];
        tiles[j].y = __builtin_bit_cast(int, ksj);
        ksm = fmaxf(ksm, ksj);
        if (a.kb != nullptr) kbm = fmaxf(kbm, a.kb[ti]);
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        kbm = fmaxf(kbm, __shfl_xor(kbm, o, 64));
        ksm = fmaxf(ksm, __shfl_xor(ksm, o, 64));
      }
      if (l == 0) {
        wmax[0][w] = kbm;
        wmax[1][w] = ksm;
      }
      if (tid == 0) redo = 0;
    }
    const float sq = S16 ? 1.f : a.qs[(int64_t)bh * a.Nb + m];
    // log2-domain score factor of key tile j: (sq * sk_j) * scale * log2(e)
    auto tile_c = [&](int j) {
      if (S16) return a.c16;
      return (sq * __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(tiles[j].y))) * a.c_log2;
    };
    // per-(b,h) buffer resources: key rows past L read as zeros (those keys are
    // masked; vt/dvt are zero there anyway), 32-bit offsets
    const auto rk8 = make_rsrc(a.k8 + qkbase * kTa, L * kTa);
    const auto rkt = make_rsrc(TAN ? reinterpret_cast<const char*>(a.kt) + (int64_t)bh * a.Nb * 16384
                                   : reinterpret_cast<const char*>(a.vt),
                               (int64_t)a.Nb * 16384);
    constexpr int kVtTile = kTa * kTa * 2 * (TAN ? 2 : 1);  // bytes per value-operand tile
    const auto rvt = make_rsrc(reinterpret_cast<const char*>(a.vt) + (int64_t)bh * a.Nb * kVtTile,
                               (int64_t)a.Nb * kVtTile);

    // ---- one pass: P = exp2(s - m), O^T += V^T P^T, dO^T += [V|dV]^T [T;P]^T ----
    // Lazy running maximum: m only moves when a tile's row maximum exceeds it
    // by more than kThr (log2 units), so P <= 2^kThr and a rescale of the
    // accumulators is rare (every row's first tile, then hardly ever).  The
    // check is one ballot per sub-tile and tile: c > 0 and rounding is
    // monotonic, so the maximum of fl(s * c) over a tile is fl(max(s) * c)
    // from the integer maximum.  With fp16 operands and the tangent, T is
    // clamped to +-60000 before its fp16 conversion as in the reference: a
    // tile whose T would reach the clamp under the lazy maximum is recomputed
    // at the exact running maximum of the wave's keys (mref), so T always
    // fits fp16 and the clamp cuts T about where an online maximum over the
    // wave's keys would (the maximum is per wave, over half the keys, and the
    // tiles go in ascending id order, so near the clamp the result depends on
    // that split and order).
    constexpr float kThr = 8.f;
    constexpr bool kClampT = TAN && T16::kDtype == SLA2H_DTYPE_F16;
    // Row sum l = sum_k p on the matrix core: acc_lm accumulates an all-ones A
    // operand times the same P^T fragments as the O^T update (one MFMA per
    // pair of tiles instead of eight VALU adds per sub-tile and tile).  The
    // JVP's mu = sum_k p dS stays an fp32 VALU sum: dO subtracts (mu / l) O
    // from a nearly equal term, so mu keeps the reference's unrounded t.
    //
    // Static shift (INT8 scores, no fp16 clamp): a per-row shift M_i at or
    // above every score of the row, fixed before the loop, replaces the
    // running maximum.  By Cauchy-Schwarz s_ij c_j <= ||q8_i|| qs ||k8_j|| ks_j
    // scale log2(e) <= ||q8_i|| qs scale log2(e) max_j kb_j (kb from
    // quant_pool).  P = 2^(s c - M_i) <= 1 then needs no maximum, no ballot and
    // no rescale, the waves of a query block share M_i (the merge adds), and
    // the softmax is unchanged by the choice of M_i.  The integer score needs
    // no conversion either: the INT8 MFMA accumulates onto C = 0x4B400000, so
    // the result read as fp32 is 1.5 * 2^23 + s exactly, and s c - M_i =
    // fl(f c - M') with M' = fl(1.5 * 2^23 c + M_i) per tile and row, whose
    // rounding moves a whole tile's exponent by at most ulp(M') / 2 < c.
    // The block falls back to the exact running maximum when a score factor
    // c exceeds 2^-9 (that shift would then reach 2^-10 log2 units), and
    // after the pass when a row's sum l fell below 2^-64 (the bound was more
    // than ~64 log2 units above the row's largest score).
    constexpr bool kStatOK = !S16 && !kClampT;
    constexpr float kMagicF = 12582912.0f;  // 1.5 * 2^23, bits 0x4B400000
    const i32x4 kMagic4 = i32x4{0x4B400000, 0x4B400000, 0x4B400000, 0x4B400000};
    f32x4 acc_lm[kQT];
    float mu_i[kQT];
    f32x4 acc_o[4][kQT], acc_do[4][kQT];  // [ct][qt]
    float mrun[kQT], mthr[kQT];  // running maximum (uniform per query column), + kThr
    float mref[kQT];  // fp16 tangent: exact running maximum of the lane's keys
    float mstat[kQT];  // static-shift pass: M_i of the lane's query column
    constexpr uint32_t kOne2 = T16::kDtype == SLA2H_DTYPE_F16 ? 0x3C003C00u : 0x3F803F80u;
    const u32x4 lm_a = u32x4{kOne2, kOne2, kOne2, kOne2};
    auto init_acc = [&](bool stat) {
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        acc_lm[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
        mu_i[qt] = 0.f;
        mrun[qt] = stat ? mstat[qt] : -INFINITY;
        mthr[qt] = -INFINITY;
        mref[qt] = -INFINITY;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          acc_o[ct][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
          acc_do[ct][qt] = acc_o[ct][qt];
        }
      }
    };

    // per-lane parts of the operand offsets of key quarter kq0 (fragment-
    // ordered tiles: each load is one contiguous 1 KB per wave); the tile base
    // and the quarter within the wave's half (sub, tangent only) are uniform
    const int k8off = (16 * kq0 + r) * kTa + 16 * g;
    const int ktoff = kq0 * 4096 + l * 16;
    const int vtoff = TAN ? kq0 * 1024 + l * 16 : kq0 * 512 + l * 8;
    auto load_keys = [&](int j, int sub, KeyRegs& kr) {
      const int n = __builtin_amdgcn_readfirstlane(tiles[j].x);
      if (!S16)
        kr.k8 = __builtin_bit_cast(i32x4, buf_load16(rk8, k8off + n * kTa * kTa, sub * 16 * kTa));
      if (TAN) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          kr.ka[ks] = buf_load16(rkt, ktoff + ks * 1024, n * 16384 + sub * 4096);
      }
    };
    auto load_vals = [&](int j, int sub, ValRegs& vr) {
      const int sb = __builtin_amdgcn_readfirstlane(tiles[j].x) * kVtTile;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        if (TAN) {
          vr.v[ct] = buf_load16(rvt, vtoff + ct * 4096, sb + sub * 1024);
        } else {
          const u32x2 x = buf_load8(rvt, vtoff + ct * 2048, sb);
          vr.v[ct] = u32x4{x.x, x.y, 0u, 0u};
        }
      }
    };

    // rescale sub-tile qt to the new running maximum max(mrun, mt) of each
    // query column; `pend` holds the previous tile's P^T fragments of a pair,
    // still to be accumulated at the old maximum
    auto rescale = [&](int qt, float mt, u32x2* pend) {
      const float mn = max_over_groups(fmaxf(mrun[qt], mt));
      const float f = mrun[qt] == -INFINITY ? 0.f : fast_exp2(mrun[qt] - mn);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        acc_o[ct][qt] *= f;
        if (TAN) acc_do[ct][qt] *= f;
      }
      acc_lm[qt] *= f;
      mu_i[qt] *= f;
      if (pend != nullptr) {
        u32x2& pp = pend[qt];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float lo = T16::to_f32((uint16_t)(pp[e] & 0xffff)) * f;
          const float hi = T16::to_f32((uint16_t)(pp[e] >> 16)) * f;
          pp[e] = pack_pair<T16>(lo, hi);
        }
      }
      mrun[qt] = mn;
      mthr[qt] = mn + kThr;
    };

    // The wave's 16 keys of one key tile (quarter kq0 + sub): scores, the
    // running-maximum check, P (and T = P dS), the mu sums and the dO^T
    // update; returns the P^T fragments for the O^T update (two quarters share
    // one K = 32 MFMA).  MASK only for the ragged prefix tail tiles (j >= T).
    auto stage = [&](const KeyRegs& kr, const ValRegs& vr, int j, int sub, u32x2 (&pb)[kQT],
                     u32x2* pend, auto mask_tag, auto stat_tag) {
      constexpr bool MASK = decltype(mask_tag)::value;
      constexpr bool STAT = decltype(stat_tag)::value && kStatOK;
      const int n = __builtin_amdgcn_readfirstlane(tiles[j].x);
      const float c = tile_c(j);
      const int64_t key0 = (int64_t)n * kTa + 16 * (kq0 + sub) + 4 * g;
      // all products of the tile first (scores of both query sub-tiles, then the
      // tangent scores), one rescale test for the tile, then the exponentials:
      // one basic block holds the MFMAs and the VALU work they overlap with
      float sv[kQT][4];  // raw scores (integer-valued for INT8)
      float mt[kQT];
      f32x4 dsv[kQT];
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        if (S16) {
          f32x4 s16 = mfma_16x16x32<T16>(kr.ka[0], qsh[qs0 + qt][2][l], f32x4{0.f, 0.f, 0.f, 0.f});
          s16 = mfma_16x16x32<T16>(kr.ka[1], qsh[qs0 + qt][3][l], s16);
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[qt][i] = s16[i];
        } else if (STAT) {
          const i32x4 si = mfma_i8_16x16x64(kr.k8, q8sh[qs0 + qt][l], kMagic4);
          // element by element through a scalar: clang's __builtin_bit_cast of
          // an ext-vector element expression reads element 0 whatever the index
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int bits = si[i];
            sv[qt][i] = __builtin_bit_cast(float, bits);
          }
        } else {
          const i32x4 si = mfma_i8_16x16x64(kr.k8, q8sh[qs0 + qt][l], i32x4{0, 0, 0, 0});
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[qt][i] = (float)si[i];
        }
      }
      if (TAN) {
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) d = mfma_16x16x32<T16>(kr.ka[ks], qsh[qs0 + qt][ks][l], d);
          dsv[qt] = d;
        }
      }
      if constexpr (!STAT) {
        bool over = false;
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          float mx = -INFINITY;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (!MASK || key0 + i < L) mx = fmaxf(mx, sv[qt][i]);
          mt[qt] = mx * c;
          over |= mt[qt] > mthr[qt];
          if (kClampT) mref[qt] = fmaxf(mref[qt], mt[qt]);
        }
        if (__builtin_amdgcn_ballot_w64(over) != 0) {
#pragma unroll
          for (int qt = 0; qt < kQT; ++qt)
            if (__builtin_amdgcn_ballot_w64(mt[qt] > mthr[qt]) != 0) rescale(qt, mt[qt], pend);
        }
      }
      float p[kQT][4], t[kQT][4];
      auto expo = [&](int qt) {
        const float moff = STAT ? fmaf(kMagicF, c, mstat[qt]) : mrun[qt];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float e = fmaf(sv[qt][i], c, -moff);
          if (MASK && key0 + i >= L) e = -INFINITY;
          p[qt][i] = fast_exp2(e);
          if (TAN) t[qt][i] = p[qt][i] * (PRE ? dsv[qt][i] : dsv[qt][i] * a.scale);
        }
      };
      if (kClampT) {
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) expo(qt);
        // a T at or past the clamp under the lazy maximum: redo the sub-tile
        // at the exact running maximum (rare)
        bool big[kQT], any = false;
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          const float tm = fmaxf(fmaxf(fabsf(t[qt][0]), fabsf(t[qt][1])),
                                 fmaxf(fabsf(t[qt][2]), fabsf(t[qt][3])));
          big[qt] = tm >= 60000.f;
          any |= big[qt];
        }
        if (__builtin_amdgcn_ballot_w64(any) != 0) {
#pragma unroll
          for (int qt = 0; qt < kQT; ++qt)
            if (__builtin_amdgcn_ballot_w64(big[qt]) != 0) {
              rescale(qt, mref[qt], pend);
              expo(qt);
            }
        }
      }
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        if (!kClampT) expo(qt);
        if (TAN) {
          float ts = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) ts += t[qt][i];
          mu_i[qt] += ts;
        }
        pb[qt].x = pack_pair<T16>(p[qt][0], p[qt][1]);
        pb[qt].y = pack_pair<T16>(p[qt][2], p[qt][3]);
        if (TAN) {
          float tc[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            tc[i] = kClampT ? fminf(fmaxf(t[qt][i], -60000.f), 60000.f) : t[qt][i];
          u32x4 bt;
          bt.x = pack_pair<T16>(tc[0], tc[1]);
          bt.y = pack_pair<T16>(tc[2], tc[3]);
          bt.z = pb[qt].x;
          bt.w = pb[qt].y;
#pragma unroll
          for (int ct = 0; ct < 4; ++ct)
            acc_do[ct][qt] = mfma_16x16x32<T16>(vr.v[ct], bt, acc_do[ct][qt]);
        }
      }
    };
    // O^T += V^T P^T for one stage (K = 16) or a pair (K = 32: the A and B
    // operand slots 4..7 take the second stage's keys 4g..4g+3)
    auto o_single = [&](const ValRegs& vr, const u32x2 (&pb)[kQT]) {
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
          acc_o[ct][qt] = mfma_16x16x16<T16>(u32x2{vr.v[ct].x, vr.v[ct].y}, pb[qt], acc_o[ct][qt]);
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt)
        acc_lm[qt] = mfma_16x16x16<T16>(u32x2{lm_a.x, lm_a.y}, pb[qt], acc_lm[qt]);
    };
    auto o_pair = [&](const ValRegs& va, const u32x2 (&pa)[kQT], const ValRegs& vb,
                      const u32x2 (&pbb)[kQT]) {
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
          acc_o[ct][qt] = mfma_16x16x32<T16>(u32x4{va.v[ct].x, va.v[ct].y, vb.v[ct].x, vb.v[ct].y},
                                             u32x4{pa[qt].x, pa[qt].y, pbb[qt].x, pbb[qt].y},
                                             acc_o[ct][qt]);
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt)
        acc_lm[qt] = mfma_16x16x32<T16>(lm_a, u32x4{pa[qt].x, pa[qt].y, pbb[qt].x, pbb[qt].y},
                                        acc_lm[qt]);
    };

    // Issue order: value loads of a stage, then the score-side prefetch of the
    // next stage -- the in-order vmcnt lets a stage wait for its own values
    // while the prefetch stays in flight.
    KeyRegs ka_, kb_;
    load_keys(0, 0, ka_);
    __syncthreads();  // key scales in tiles[].y, block maxima in wmax
    // Per-block choice of the static shift (uniform): kb given, every score
    // factor c_j <= 2^-9; M_i = ||q8_i|| qs scale log2(e) max_j kb_j.
    bool exact = true;
    if (kStatOK && a.kb != nullptr) {
      const float kbm = fmaxf(fmaxf(wmax[0][0], wmax[0][1]), fmaxf(wmax[0][2], wmax[0][3]));
      const float ksm = fmaxf(fmaxf(wmax[1][0], wmax[1][1]), fmaxf(wmax[1][2], wmax[1][3]));
      const float cq = sq * a.c_log2;
      exact = !(cq * ksm <= 0x1p-9f);
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        // ||q8_i||^2 of query column r of sub-tile qs0 + qt: 16 bytes per lane
        // group, summed over the four groups (integers below 2^21: exact)
        const i32x4 v = q8sh[qs0 + qt][l];
        int n2 = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) n2 = __builtin_amdgcn_sdot4(v[e], v[e], n2, false);
        mstat[qt] = __builtin_sqrtf(sum_over_groups((float)n2)) * cq * kbm;
      }
    }
    for (;;) {  // passes: static shift, or (first or after an underflow) exact maximum
    init_acc(!exact);
    int j = 0;
    auto run_tiles = [&](auto stat_tag) {
    if (TAN) {
      // both quarters of the wave's key half of every tile, as one pair
      auto tile_pair = [&](int jt, auto mask_tag) {
        ValRegs va, vb;
        u32x2 pa[kQT], pbb[kQT];
        load_vals(jt, 0, va);
        load_keys(jt, 1, kb_);
        stage(ka_, va, jt, 0, pa, nullptr, mask_tag, stat_tag);
        load_vals(jt, 1, vb);
        load_keys(jt + 1 < J ? jt + 1 : J - 1, 0, ka_);
        stage(kb_, vb, jt, 1, pbb, pa, mask_tag, stat_tag);
        o_pair(va, pa, vb, pbb);
      };
      for (; j < Tu; ++j) tile_pair(j, std::false_type{});  // routed video tiles
      for (; j < J; ++j) tile_pair(j, std::true_type{});    // ragged prefix tails
    } else {
      // routed video tiles in pairs (full, unmasked); the two tiles' V
      // fragments load straight into the slots 0..3 and 4..7 of one K = 32
      // operand (the primal stage itself reads no values)
      for (; j + 1 < Tu; j += 2) {
        u32x4 vp[4];
        u32x2 pa[kQT], pbb[kQT];
        auto load_v = [&](int jt, int slot) {
          const int sb = __builtin_amdgcn_readfirstlane(tiles[jt].x) * kVtTile;
#pragma unroll
          for (int ct = 0; ct < 4; ++ct) {
            const u32x2 x = buf_load8(rvt, vtoff + ct * 2048, sb);
            vp[ct][2 * slot] = x.x;
            vp[ct][2 * slot + 1] = x.y;
          }
        };
        load_v(j, 0);
        load_keys(j + 1, 0, kb_);
        stage(ka_, ValRegs{}, j, 0, pa, nullptr, std::false_type{}, stat_tag);
        load_v(j + 1, 1);
        load_keys(j + 2 < J ? j + 2 : J - 1, 0, ka_);
        stage(kb_, ValRegs{}, j + 1, 0, pbb, pa, std::false_type{}, stat_tag);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
          for (int qt = 0; qt < kQT; ++qt)
            acc_o[ct][qt] = mfma_16x16x32<T16>(vp[ct], u32x4{pa[qt].x, pa[qt].y, pbb[qt].x, pbb[qt].y},
                                               acc_o[ct][qt]);
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
          acc_lm[qt] = mfma_16x16x32<T16>(lm_a, u32x4{pa[qt].x, pa[qt].y, pbb[qt].x, pbb[qt].y},
                                          acc_lm[qt]);
      }
      // odd leftover routed tile and the ragged prefix tail tiles, one at a time
      for (; j < J; ++j) {
        ValRegs vr;
        u32x2 pb[kQT];
        load_vals(j, 0, vr);
        load_keys(j + 1 < J ? j + 1 : J - 1, 0, kb_);
        if (j < Tu)
          stage(ka_, vr, j, 0, pb, nullptr, std::false_type{}, stat_tag);
        else
          stage(ka_, vr, j, 0, pb, nullptr, std::true_type{}, stat_tag);
        o_single(vr, pb);
        ka_ = kb_;
      }
    }
    };
    if (!kStatOK || exact)
      run_tiles(std::false_type{});
    else
      run_tiles(std::true_type{});
    // Lane indices for the merge and epilogue, re-derived from vtoff (live
    // through the key loop anyway; the empty asm keeps the compiler from
    // folding it back): l, r and g themselves then need no register across
    // the loop.
    {
      int lt = vtoff;
      asm volatile("" : "+v"(lt));
      const int l = (lt - (TAN ? kq0 * 1024 : kq0 * 512)) >> (TAN ? 4 : 3);
      const int r = l & 15, g = l >> 4;

      // The wave finalises block sub-tile qo over all four output column tiles:
      // primal only its own sub-tile w, with the tangent sub-tile qs0 + (w & 1)
      // of its query half (the partner wave w ^ 1 takes the other).  The
      // complement record is requested now (in flight through the merge): the
      // zc, dzc parts by every wave, the Hc, dHc fragments of column tile w by
      // wave w, which splits them once for the workgroup after the merge.
      constexpr int kNcc = 4;
      const int kh = w & 1;  // tangent: the wave's key half and finalised sub-tile qs0 + kh
      const int qo = TAN ? qs0 + kh : w;
      // [ks][Hc, dHc][j]: H[32 ks + 8 g + j][16 w + r]
      float hraw[2][TAN ? 2 : 1][8];
      f32x4 zraw[2][2][2];     // [ks][zc, dzc][half]: z[32 ks + 8 g + 4 half ..]
      const float* rec = reinterpret_cast<const float*>(a.comp + ((int64_t)bh * a.Mq + mq) * kRec);
      auto load_h = [&](int cc) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int mat = 0; mat < (TAN ? 2 : 1); ++mat)
#pragma unroll
            for (int jj = 0; jj < 8; ++jj)
              hraw[ks][mat][jj] = rec[4096 * mat + (32 * ks + 8 * g + jj) * 64 + 16 * cc + r];
      };
      if (LINEAR) {
        load_h(w);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int mat = 0; mat < (TAN ? 2 : 1); ++mat)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
              zraw[ks][mat][hf] = *reinterpret_cast<const f32x4*>(rec + 8192 + 64 * mat + 32 * ks + 8 * g + 4 * hf);
      }
      float l_i[kQT];
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        l_i[qt] = acc_lm[qt][0];  // every row of the product holds the column sum
        if (TAN) mu_i[qt] = sum_over_groups(mu_i[qt]);
      }

      // ---- merge the per-wave states (fixed order: deterministic) ----
      __syncthreads();  // every wave is done with the sort's use of mbuf
      if (g == 0) {
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          stat[0][w][qt][r] = mrun[qt];
          stat[1][w][qt][r] = l_i[qt];
          stat[2][w][qt][r] = mu_i[qt];
        }
      }
      __syncthreads();
      // waves holding parts of the same queries: the pair w0, w0 + 1 of the
      // query half with the tangent, all four primal only
      constexpr int kNw = TAN ? 2 : 4;
      const int w0 = TAN ? (w & ~1) : 0;
      const int qsel = TAN ? kh : qo;  // the finalised sub-tile among the wave's own
      float fself[kQT];
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < kNw; ++ww) M = fmaxf(M, stat[0][w0 + ww][qt][r]);
        fself[qt] = (mrun[qt] == -INFINITY) ? 0.f : fast_exp2(mrun[qt] - M);
      }
      float Mw = -INFINITY;
#pragma unroll
      for (int ww = 0; ww < kNw; ++ww) Mw = fmaxf(Mw, stat[0][w0 + ww][qsel][r]);
      float ltot = 0.f, mutot = 0.f;
#pragma unroll
      for (int ww = 0; ww < kNw; ++ww) {
        const float mw = stat[0][w0 + ww][qsel][r];
        const float f = (mw == -INFINITY) ? 0.f : fast_exp2(mw - Mw);
        ltot += stat[1][w0 + ww][qsel][r] * f;
        mutot += stat[2][w0 + ww][qsel][r] * f;
      }
      // static shift: a row sum below 2^-64 sends the block to the exact pass
      // (read after the merge's barriers below)
      if (!exact && !(ltot >= 0x1p-64f)) redo = 1;

      f32x4 O[kNcc], DO[kNcc];
      if (TAN) {
        // hand the partner its sub-tile (the wave's other one, 1 - kh), scaled to
        // the pair's maximum; add the partner's part of sub-tile kh to our own.
        // Values are picked, never addressed, by kh: register arrays indexed by
        // a runtime value would move to scratch memory.
        auto pick = [](bool c, auto x, auto y) { return c ? x : y; };
        const bool k1 = kh != 0;
        const float fo = pick(k1, fself[0], fself[1]);
        const float fm = pick(k1, fself[1], fself[0]);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          *reinterpret_cast<f32x4*>(&mbuf[w][2 * ct][l][0]) = pick(k1, acc_o[ct][0], acc_o[ct][1]) * fo;
          *reinterpret_cast<f32x4*>(&mbuf[w][2 * ct + 1][l][0]) =
              pick(k1, acc_do[ct][0], acc_do[ct][1]) * fo;
        }
        __syncthreads();
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          O[ct] = pick(k1, acc_o[ct][1], acc_o[ct][0]) * fm +
                  *reinterpret_cast<const f32x4*>(&mbuf[w ^ 1][2 * ct][l][0]);
          DO[ct] = pick(k1, acc_do[ct][1], acc_do[ct][0]) * fm +
                   *reinterpret_cast<const f32x4*>(&mbuf[w ^ 1][2 * ct + 1][l][0]);
        }
      } else {
        // two rounds (column tiles 0-1, then 2-3); every wave sums its sub-tile
#pragma unroll
        for (int rd = 0; rd < 2; ++rd) {
#pragma unroll
          for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int qt = 0; qt < kQT; ++qt)
              *reinterpret_cast<f32x4*>(&mbuf[w][4 * cc + qt][l][0]) = acc_o[2 * rd + cc][qt] * fself[qt];
          __syncthreads();
#pragma unroll
          for (int cc = 0; cc < 2; ++cc) {
            f32x4 so = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ww = 0; ww < 4; ++ww) so += *reinterpret_cast<const f32x4*>(&mbuf[ww][4 * cc + qo][l][0]);
            O[2 * rd + cc] = so;
          }
          if (rd == 0) __syncthreads();
        }
      }

      if (!exact && redo != 0) {  // uniform: written before the merge's barriers
        exact = true;
        load_keys(0, 0, ka_);
        continue;
      }

      // ---- Hc (dHc) as bf16 hi/lo A-operand fragments in LDS, in the
      // merge buffer (free again): wave w splits column tile w once for the
      // workgroup; entry [mat][ct][ks][hi, lo][lane] is the u32x4 lane l uses ----
      u32x4* hfrag = reinterpret_cast<u32x4*>(&mbuf[0][0][0][0]);
      auto hidx = [&](int mat, int ct, int ks, int part) {
        return (((mat * 4 + ct) * 2 + ks) * 2 + part) * 64 + l;
      };
      if (LINEAR) {
        __syncthreads();  // every wave has read its merge inputs
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int mat = 0; mat < (TAN ? 2 : 1); ++mat) {
            u32x4 hi, lo;
            split_hfrag(hraw[ks][mat], hi, lo);
            hfrag[hidx(mat, w, ks, 0)] = hi;
            hfrag[hidx(mat, w, ks, 1)] = lo;
          }
        __syncthreads();
      }

      // ---- epilogue: query q0 + 16 qo + r, output columns 16 cc + 4g + i ----
      // the lane's row within the block; the block's rows inside L are reached
      // through buffer resources (SGPR base, 32-bit offsets, rows past L read as
      // zeros and are not written), so no 64-bit lane address is formed here
      const int erow = 16 * qo + r;
      const int brows = (int)(L - q0 < kTa ? L - q0 : kTa);
      const float rl = 1.f / ltot;
      const float inv_mu = mutot * rl;
      f32x4 os[kNcc], dos[kNcc];
#pragma unroll
      for (int cc = 0; cc < kNcc; ++cc) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          os[cc][i] = O[cc][i] * rl;
          if (TAN) dos[cc][i] = DO[cc][i] * rl - inv_mu * os[cc][i];
        }
      }

      if (LINEAR) {
        // phi(q), dphi(q) of this lane's query in B-operand layout: d = 32 ks + 8 g + e
        float qv[2][8], dqv[2][8];
        const auto rq = make_rsrc(a.q + blk, (int64_t)brows * kTa * 2);
        // tangent: the [dQ|Q] operand fragments in LDS are exactly this lane's
        // row (zero past L), scaled by the power-of-two softmax scale when PRE
        const float unscale = PRE ? 1.f / a.scale : 1.f;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          u32x4 u, du = u32x4{0, 0, 0, 0};
          if (TAN) {
            u = qsh[qo][2 + ks][l];
            du = qsh[qo][ks][l];
          } else {
            u = buf_load16(rq, (erow * kTa + 32 * ks + 8 * g) * 2, 0);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            qv[ks][2 * e] = T16::to_f32((uint16_t)(u[e] & 0xffff)) * unscale;
            qv[ks][2 * e + 1] = T16::to_f32((uint16_t)(u[e] >> 16)) * unscale;
            dqv[ks][2 * e] = T16::to_f32((uint16_t)(du[e] & 0xffff)) * unscale;
            dqv[ks][2 * e + 1] = T16::to_f32((uint16_t)(du[e] >> 16)) * unscale;
          }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e) mx = fmaxf(mx, qv[ks][e]);
        mx = max_over_groups(mx);
        float den = 0.f;
        float phi[2][8], dphi[2][8];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            phi[ks][e] = __expf(qv[ks][e] - mx);
            den += phi[ks][e];
          }
        den = sum_over_groups(den);
        const float rden = 1.f / den;
        float qdot = 0.f;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            phi[ks][e] = phi[ks][e] * rden;
            qdot += phi[ks][e] * dqv[ks][e];
          }
        if (TAN) {
          qdot = sum_over_groups(qdot);
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) dphi[ks][e] = phi[ks][e] * (dqv[ks][e] - qdot);
        }
        // bf16 hi/lo operand halves
        u32x4 ph[2], pl[2], dph[2], dpl[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a0 = phi[ks][2 * e], a1 = phi[ks][2 * e + 1];
            ph[ks][e] = pack_pair<BF16>(a0, a1);
            pl[ks][e] = pack_pair<BF16>(a0 - bf16_val((uint16_t)(ph[ks][e] & 0xffff)),
                                        a1 - bf16_val((uint16_t)(ph[ks][e] >> 16)));
            if (TAN) {
              const float b0 = dphi[ks][2 * e], b1 = dphi[ks][2 * e + 1];
              dph[ks][e] = pack_pair<BF16>(b0, b1);
              dpl[ks][e] = pack_pair<BF16>(b0 - bf16_val((uint16_t)(dph[ks][e] & 0xffff)),
                                           b1 - bf16_val((uint16_t)(dph[ks][e] >> 16)));
            }
          }
        }
        float dn = 0.f, ddn = 0.f;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float z = zraw[ks][0][e >> 2][e & 3];
            dn += phi[ks][e] * z;
            if (TAN) ddn += dphi[ks][e] * z + phi[ks][e] * zraw[ks][1][e >> 2][e & 3];
          }
        }
        dn = sum_over_groups(dn);
        dn = dn >= 0.f ? dn + a.eps_l : dn - a.eps_l;
        const float rdn = 1.f / dn;
        if (TAN) ddn = sum_over_groups(ddn);
        const float al = a.alpha[(int64_t)h * a.alpha_stride + mq];
#pragma unroll
        for (int cc = 0; cc < kNcc; ++cc) {
          f32x4 num = f32x4{0.f, 0.f, 0.f, 0.f}, dnum = num;
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const u32x4 hh = hfrag[hidx(0, cc, ks, 0)], hl = hfrag[hidx(0, cc, ks, 1)];
            num = mfma_bf16_16x16x32(hh, ph[ks], num);
            num = mfma_bf16_16x16x32(hh, pl[ks], num);
            num = mfma_bf16_16x16x32(hl, ph[ks], num);
            if (TAN) {
              const u32x4 dh = hfrag[hidx(1, cc, ks, 0)], dl = hfrag[hidx(1, cc, ks, 1)];
              dnum = mfma_bf16_16x16x32(hh, dph[ks], dnum);
              dnum = mfma_bf16_16x16x32(hh, dpl[ks], dnum);
              dnum = mfma_bf16_16x16x32(hl, dph[ks], dnum);
              dnum = mfma_bf16_16x16x32(dh, ph[ks], dnum);
              dnum = mfma_bf16_16x16x32(dh, pl[ks], dnum);
              dnum = mfma_bf16_16x16x32(dl, ph[ks], dnum);
            }
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float ol = num[i] * rdn;
            os[cc][i] = al * os[cc][i] + (1.f - al) * ol;
            if (TAN) {
              const float dol = (dnum[i] - ol * ddn) * rdn;
              dos[cc][i] = al * dos[cc][i] + (1.f - al) * dol;
            }
          }
        }
      }

      {
        const auto ro_ = make_rsrc(a.o + blk, (int64_t)brows * kTa * 4);
        const auto rdo = make_rsrc(TAN ? a.dout + blk : a.o + blk, (int64_t)brows * kTa * 4);
        const int oo = (erow * kTa + 4 * g) * 4;
#pragma unroll
        for (int cc = 0; cc < kNcc; ++cc) {
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, os[cc]), ro_, oo + 64 * cc, 0, 0);
          if (TAN)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, dos[cc]), rdo, oo + 64 * cc, 0, 0);
        }
      }
    }
    break;
    }  // pass loop
    if (!TAN) break;
  }  // unit loop
}

// Grid of the fused kernel: with the tangent, two persistent workgroups per
// CU (the occupancy its registers allow) in every XCD, else one workgroup per
// unit.  The CU count is read once per device.
static int fwd_grid(int64_t per_xcd, bool tan, int* nblocks) {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cus[kMaxDev];
  int slots = (int)per_xcd;
  if (tan) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return (int)err;
    if (dev < 0 || dev >= kMaxDev) return (int)hipErrorInvalidDevice;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n == 0) {
      err = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
      if (err != hipSuccess) return (int)err;
      cus[dev].store(n, std::memory_order_relaxed);
    }
    const int per = 2 * n / 8 > 0 ? 2 * n / 8 : 1;  // resident workgroups per XCD
    if (per < slots) slots = per;
  }
  *nblocks = 8 * slots;
  return 0;
}

template <typename T16, bool PRE>
static void launch_fwd(const FwdArgs& a, bool tan, bool linear, int nblocks, hipStream_t st) {
  if (tan && linear)
    fwd_jvp_kernel<T16, true, true, PRE, false><<<nblocks, 256, 0, st>>>(a);
  else if (tan)
    fwd_jvp_kernel<T16, true, false, PRE, false><<<nblocks, 256, 0, st>>>(a);
  else if (linear)
    fwd_jvp_kernel<T16, false, true, false, false><<<nblocks, 256, 0, st>>>(a);
  else
    fwd_jvp_kernel<T16, false, false, false, false><<<nblocks, 256, 0, st>>>(a);
}

}  // namespace sla2h

using namespace sla2h;

extern "C" int sla2h_fwd_jvp(const void* q, const void* dq, const void* kt, const void* vt,
                             const int8_t* q8, const int8_t* k8,
                             const float* qs, const float* ks, const float* kb, const void* comp,
                             const float* alpha, int alpha_stride, const int32_t* lut, int dtype,
                             int B, int H, int64_t L, int D, int E, int Np, int T, float scale,
                             float eps_l, int flags, float* o, float* dout, void* stream) {
  SLA2H_CHECK_ARG(q && vt && q8 && k8 && qs && ks && lut && o);
  SLA2H_CHECK_ARG(D == kTa && E == kTa);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && L > 0 && Np > 0 && (int64_t)Np * E <= L);
  SLA2H_CHECK_ARG(T >= 1 && T <= Np);
  SLA2H_CHECK_ARG(scale > 0.f);  // the tile-maximum pass relies on positive score factors
  const int Nb_ = (int)((L + E - 1) / E);
  SLA2H_CHECK_ARG(T + (Nb_ - Np) <= kMaxTiles);
  const bool tan = dq != nullptr;
  if (tan) SLA2H_CHECK_ARG(kt && dout);
  const bool linear = (flags & SLA2H_FLAG_SPARSE_ONLY) == 0;
  if (linear) SLA2H_CHECK_ARG(comp && alpha && alpha_stride >= 0);
  const int Nb = (int)((L + E - 1) / E);
  const int64_t nwork = (int64_t)Nb * B * H;  // query blocks
  const int64_t per_xcd = (nwork + 7) / 8;
  SLA2H_CHECK_ARG(8 * per_xcd < (1ll << 31));
  FwdArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.dq = static_cast<const uint16_t*>(dq);
  a.kt = static_cast<const uint16_t*>(kt);
  a.vt = static_cast<const uint16_t*>(vt);
  a.q8 = q8;
  a.k8 = k8;
  a.qs = qs;
  a.ks = ks;
  a.kb = kb;
  a.comp = static_cast<const unsigned char*>(comp);
  a.alpha = alpha;
  a.lut = lut;
  a.o = o;
  a.dout = dout;
  a.L = L;
  a.H = H;
  a.Nb = Nb;
  a.Np = Np;
  a.Mb = Nb;
  a.T = T;
  a.n_tail = Nb - Np;
  a.alpha_stride = alpha_stride;
  a.nwork = (int)nwork;
  a.per_xcd = (int)per_xcd;
  a.scale = scale;
  {
    int ex;
    const float fr = frexpf(scale, &ex);
    a.prescale = (fr == 0.5f && ex > -100 && ex < 100) ? 1 : 0;
  }
  a.c_log2 = scale * 1.4426950408889634f;
  a.c16 = a.c_log2;
  a.eps_l = eps_l;
  a.qshift = 0;
  a.Mq = Nb;
  a.ragged = -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int nblocks = 0;
  if (const int e = fwd_grid(per_xcd, tan, &nblocks)) return e;
  if (dtype == SLA2H_DTYPE_BF16) {
    if (a.prescale)
      launch_fwd<BF16, true>(a, tan, linear, nblocks, st);
    else
      launch_fwd<BF16, false>(a, tan, linear, nblocks, st);
  } else {
    launch_fwd<F16, false>(a, tan, linear, nblocks, st);
  }
  return (int)hipGetLastError();
}

extern "C" int sla2h_fwd_jvp_1d(const void* q, const void* dq, const void* kt, const void* vt,
                                const void* comp, const float* alpha, int alpha_stride,
                                const int32_t* lut, int dtype, int B, int H, int64_t L, int D,
                                int bq, int bk, int T, float scale, float eps_l, float* o,
                                float* dout, void* stream) {
  SLA2H_CHECK_ARG(q && dq && kt && vt && comp && alpha && lut && o && dout);
  SLA2H_CHECK_ARG(D == kTa && bk == kTa && alpha_stride >= 0);
  SLA2H_CHECK_ARG(bq == 64 || bq == 128 || bq == 256);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && L > 0 && scale > 0.f);
  const int Nb = (int)((L + bk - 1) / bk);
  SLA2H_CHECK_ARG(T >= 1 && T <= Nb && T <= kMaxTiles);
  const int64_t nwork = (int64_t)Nb * B * H;  // 64-row query blocks
  const int64_t per_xcd = (nwork + 7) / 8;
  SLA2H_CHECK_ARG(8 * per_xcd < (1ll << 31));
  FwdArgs a = {};
  a.q = static_cast<const uint16_t*>(q);
  a.dq = static_cast<const uint16_t*>(dq);
  a.kt = static_cast<const uint16_t*>(kt);
  a.vt = static_cast<const uint16_t*>(vt);
  a.comp = static_cast<const unsigned char*>(comp);
  a.alpha = alpha;
  a.lut = lut;
  a.o = o;
  a.dout = dout;
  a.L = L;
  a.H = H;
  a.Nb = Nb;
  a.Np = Nb;
  a.Mb = Nb;
  a.T = T;
  a.n_tail = 0;
  a.alpha_stride = alpha_stride;
  a.nwork = (int)nwork;
  a.per_xcd = (int)per_xcd;
  a.scale = scale;
  {
    int ex;
    const float fr = frexpf(scale, &ex);
    a.prescale = (fr == 0.5f && ex > -100 && ex < 100) ? 1 : 0;
  }
  a.c_log2 = scale * 1.4426950408889634f;
  a.eps_l = eps_l;
  a.qshift = bq == 64 ? 0 : (bq == 128 ? 1 : 2);
  a.Mq = (int)((L + bq - 1) / bq);
  a.ragged = (L % kTa) ? Nb - 1 : -1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int nblocks = 0;
  if (const int e = fwd_grid(per_xcd, true, &nblocks)) return e;
  if (dtype == SLA2H_DTYPE_BF16 && a.prescale) {
    a.c16 = 1.4426950408889634f;  // the Q operands carry the scale
    fwd_jvp_kernel<BF16, true, true, true, true><<<nblocks, 256, 0, st>>>(a);
  } else if (dtype == SLA2H_DTYPE_BF16) {
    a.c16 = a.c_log2;
    fwd_jvp_kernel<BF16, true, true, false, true><<<nblocks, 256, 0, st>>>(a);
  } else {
    a.c16 = a.c_log2;
    fwd_jvp_kernel<F16, true, true, false, true><<<nblocks, 256, 0, st>>>(a);
  }
  return (int)hipGetLastError();
}
