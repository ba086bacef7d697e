// Fused SLA2 sparse + linear attention with forward-mode JVP, gfx950.
//
// One workgroup (4 wave64) per (query block m, b, h): 64 query rows.  The key
// tiles of the block (T routed video tiles + n_tail prefix blocks) are split
// across the waves by key: wave w owns keys 16w..16w+15 of every tile and runs
// its own online softmax over them for all 64 queries; the four partial
// softmax states are merged once at the end through LDS.  Each wave therefore
// streams only its quarter of every key tile straight from global memory
// into MFMA operand registers -- no LDS staging, no barriers in the loop.
//
// Scores are computed transposed (S^T = K Q^T) so that a lane holds one query
// column: the S^T output fragment is directly the B operand of
// O^T = V^T P^T, and the per-query softmax statistics stay lane-resident.
//
// Reference semantics: models/sla2_cube_qat.py:448-602 (_cube_fused_jvp_kernel),
// sparse-only variant :59-169 (_sla2_cube_jvp_qat_kernel).
#include "common.h"

namespace sla2h {

constexpr int kTa = 64;
constexpr size_t kRec = 2 * 16384 + 2 * 256;

struct FwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* dq;
  const uint16_t* dk;
  const uint16_t* vt;
  const uint16_t* dvt;
  const int8_t* q8;
  const int8_t* k8;
  const float* qs;
  const float* ks;
  const unsigned char* comp;
  const float* alpha;
  const int32_t* lut;
  float* o;
  float* dout;
  int64_t L;
  int H, Nb, Np, Mb, T, n_tail, alpha_stride;
  float scale, c_log2, eps_l;
};

struct KeyRegs {
  i32x4 k8;      // K8[key 16w + r][16g .. 16g+15]
  u32x4 ka[4];   // ks 0,1: K[key][32ks + 8g ..], ks 2,3: dK[key][32(ks-2) + 8g ..]
  u32x2 va[4];   // Vt[c = 16ct + r][keys 16w + 4g .. +3]
  u32x2 dva[4];
  float sk;
  int n;
};

template <typename T16, bool TAN, bool LINEAR>
__global__ __launch_bounds__(256, 1) void fwd_jvp_kernel(FwdArgs a) {
  __shared__ float stat[3][4][4][16];            // [m,l,mu][wave][qt][r]
  __shared__ __align__(16) float xbuf[4][4][64][4];  // [wave][qt][lane][i]

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, r = l & 15, g = l >> 4;
  const int m = blockIdx.x % a.Mb;
  const int bh = blockIdx.x / a.Mb;
  const int h = bh % a.H;
  const int64_t L = a.L;
  const int64_t qkbase = (int64_t)bh * L;

  // ---- query-side MFMA B operands for the 4 query sub-tiles ----
  i32x4 q8b[4];
  u32x4 qb[4][4];
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    const int64_t row = (int64_t)m * kTa + 16 * qt + r;
    const bool ok = row < L;
    const int64_t ro = (qkbase + row) * kTa;
    q8b[qt] = ok ? *reinterpret_cast<const i32x4*>(a.q8 + ro + 16 * g) : i32x4{0, 0, 0, 0};
    if (TAN) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        qb[qt][ks] = ok ? *reinterpret_cast<const u32x4*>(a.dq + ro + 32 * ks + 8 * g)
                        : u32x4{0, 0, 0, 0};
        qb[qt][ks + 2] = ok ? *reinterpret_cast<const u32x4*>(a.q + ro + 32 * ks + 8 * g)
                            : u32x4{0, 0, 0, 0};
      }
    }
  }
  const float sq = a.qs[(int64_t)bh * a.Nb + m];

  float m_i[4], l_i[4], mu_i[4];
  f32x4 acc_o[4][4], acc_do[4][4];  // [ct][qt]
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    m_i[qt] = -INFINITY;
    l_i[qt] = 0.f;
    mu_i[qt] = 0.f;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      acc_o[ct][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
      acc_do[ct][qt] = acc_o[ct][qt];
    }
  }

  const int32_t* lrow = a.lut + ((int64_t)bh * a.Mb + m) * a.T;
  const int J = a.T + a.n_tail;

  auto load_keys = [&](int j, KeyRegs& kr) {
    int n = j < a.T ? lrow[j] : a.Np + (j - a.T);
    if ((unsigned)n >= (unsigned)a.Nb) n = -1;  // corrupt id: skipped
    kr.n = n;
    if (n < 0) return;
    const int64_t krow = (int64_t)n * kTa + 16 * w + r;
    const bool ok = krow < L;
    const int64_t ko = (qkbase + krow) * kTa;
    kr.sk = a.ks[(int64_t)bh * a.Nb + n];
    kr.k8 = ok ? *reinterpret_cast<const i32x4*>(a.k8 + ko + 16 * g) : i32x4{0, 0, 0, 0};
    if (TAN) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        kr.ka[ks] = ok ? *reinterpret_cast<const u32x4*>(a.k + ko + 32 * ks + 8 * g)
                       : u32x4{0, 0, 0, 0};
        kr.ka[ks + 2] = ok ? *reinterpret_cast<const u32x4*>(a.dk + ko + 32 * ks + 8 * g)
                           : u32x4{0, 0, 0, 0};
      }
    }
    const int64_t vo = ((int64_t)bh * a.Nb + n) * kTa * kTa + 16 * w + 4 * g;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      kr.va[ct] = *reinterpret_cast<const u32x2*>(a.vt + vo + (16 * ct + r) * kTa);
      if (TAN) kr.dva[ct] = *reinterpret_cast<const u32x2*>(a.dvt + vo + (16 * ct + r) * kTa);
    }
  };

  KeyRegs cur, nxt;
  if (J > 0) load_keys(0, cur);
  for (int j = 0; j < J; ++j) {
    if (j + 1 < J) load_keys(j + 1, nxt);
    if (cur.n >= 0) {
      const float sqk = sq * cur.sk;
      const int64_t key0 = (int64_t)cur.n * kTa + 16 * w + 4 * g;
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
        const i32x4 si = mfma_i8_16x16x64(cur.k8, q8b[qt], i32x4{0, 0, 0, 0});
        float s2[4], p[4], ds[4], t[4];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float sf = (float)si[i] * sqk;
          s2[i] = (key0 + i < L) ? sf * a.c_log2 : -INFINITY;
          mx = fmaxf(mx, s2[i]);
        }
        if (TAN) {
          f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) d = mfma_16x16x32<T16>(cur.ka[ks], qb[qt][ks], d);
#pragma unroll
          for (int i = 0; i < 4; ++i) ds[i] = d[i] * a.scale;
        }
        mx = max_over_groups(mx);
        const float m_new = fmaxf(m_i[qt], mx);
        const bool dead = m_new == -INFINITY;
        const float al = dead ? 1.f : exp2f(m_i[qt] - m_new);
        float ps = 0.f, ts = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = dead ? 0.f : exp2f(s2[i] - m_new);
          ps += p[i];
          if (TAN) {
            t[i] = p[i] * ds[i];
            ts += t[i];
          }
        }
        ps = sum_over_groups(ps);
        l_i[qt] = l_i[qt] * al + ps;
        if (TAN) {
          ts = sum_over_groups(ts);
          mu_i[qt] = mu_i[qt] * al + ts;
        }
        m_i[qt] = m_new;

        u32x2 pb;
        pb.x = pack2(T16::from_f32(p[0]), T16::from_f32(p[1]));
        pb.y = pack2(T16::from_f32(p[2]), T16::from_f32(p[3]));
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          acc_o[ct][qt] = acc_o[ct][qt] * al;
          acc_o[ct][qt] = mfma_16x16x16<T16>(cur.va[ct], pb, acc_o[ct][qt]);
        }
        if (TAN) {
          float tc[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            tc[i] = (T16::kDtype == SLA2H_DTYPE_F16) ? fminf(fmaxf(t[i], -60000.f), 60000.f) : t[i];
          u32x4 bt;
          bt.x = pack2(T16::from_f32(tc[0]), T16::from_f32(tc[1]));
          bt.y = pack2(T16::from_f32(tc[2]), T16::from_f32(tc[3]));
          bt.z = pb.x;
          bt.w = pb.y;
#pragma unroll
          for (int ct = 0; ct < 4; ++ct) {
            u32x4 av;
            av.x = cur.va[ct].x;
            av.y = cur.va[ct].y;
            av.z = cur.dva[ct].x;
            av.w = cur.dva[ct].y;
            acc_do[ct][qt] = acc_do[ct][qt] * al;
            acc_do[ct][qt] = mfma_16x16x32<T16>(av, bt, acc_do[ct][qt]);
          }
        }
      }
    }
    cur = nxt;
  }

  // ---- merge the four per-wave softmax states (fixed order: exact ties) ----
  if (g == 0) {
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
      stat[0][w][qt][r] = m_i[qt];
      stat[1][w][qt][r] = l_i[qt];
      stat[2][w][qt][r] = mu_i[qt];
    }
  }
  __syncthreads();
  float fself[4];
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, stat[0][ww][qt][r]);
    fself[qt] = (m_i[qt] == -INFINITY) ? 0.f : exp2f(m_i[qt] - M);
  }
  float Mw = -INFINITY;
#pragma unroll
  for (int ww = 0; ww < 4; ++ww) Mw = fmaxf(Mw, stat[0][ww][w][r]);
  float ltot = 0.f, mutot = 0.f;
#pragma unroll
  for (int ww = 0; ww < 4; ++ww) {
    const float mw = stat[0][ww][w][r];
    const float f = (mw == -INFINITY) ? 0.f : exp2f(mw - Mw);
    ltot += stat[1][ww][w][r] * f;
    mutot += stat[2][ww][w][r] * f;
  }

  f32x4 O[4], DO[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
#pragma unroll
    for (int qt = 0; qt < 4; ++qt)
      *reinterpret_cast<f32x4*>(&xbuf[w][qt][l][0]) = acc_o[ct][qt] * fself[qt];
    __syncthreads();
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) s += *reinterpret_cast<const f32x4*>(&xbuf[ww][w][l][0]);
    O[ct] = s;
    __syncthreads();
    if (TAN) {
#pragma unroll
      for (int qt = 0; qt < 4; ++qt)
        *reinterpret_cast<f32x4*>(&xbuf[w][qt][l][0]) = acc_do[ct][qt] * fself[qt];
      __syncthreads();
      f32x4 s2 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) s2 += *reinterpret_cast<const f32x4*>(&xbuf[ww][w][l][0]);
      DO[ct] = s2;
      __syncthreads();
    }
  }

  // ---- epilogue for queries 16w + r of this block ----
  const int64_t qrow = (int64_t)m * kTa + 16 * w + r;
  const float inv_mu = mutot / ltot;
  f32x4 os[4], dos[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      os[ct][i] = O[ct][i] / ltot;
      if (TAN) dos[ct][i] = DO[ct][i] / ltot - inv_mu * os[ct][i];
    }
  }

  if (LINEAR) {
    // phi(q), dphi(q) for query qrow in B-operand layout: d = 32 ks + 8 g + jj
    float qv[2][8], dqv[2][8];
    const bool qok = qrow < L;
    const int64_t ro = (qkbase + qrow) * kTa;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4 u = qok ? *reinterpret_cast<const u32x4*>(a.q + ro + 32 * ks + 8 * g) : u32x4{0, 0, 0, 0};
      u32x4 du = u32x4{0, 0, 0, 0};
      if (TAN && qok) du = *reinterpret_cast<const u32x4*>(a.dq + ro + 32 * ks + 8 * g);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qv[ks][2 * e] = T16::to_f32((uint16_t)(u[e] & 0xffff));
        qv[ks][2 * e + 1] = T16::to_f32((uint16_t)(u[e] >> 16));
        dqv[ks][2 * e] = T16::to_f32((uint16_t)(du[e] & 0xffff));
        dqv[ks][2 * e + 1] = T16::to_f32((uint16_t)(du[e] >> 16));
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
    float qdot = 0.f;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        phi[ks][e] = phi[ks][e] / den;
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
      uint16_t hi[8], lo[8], dhi[8], dlo[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        hi[e] = bf16_bits(phi[ks][e]);
        lo[e] = bf16_bits(phi[ks][e] - bf16_val(hi[e]));
        if (TAN) {
          dhi[e] = bf16_bits(dphi[ks][e]);
          dlo[e] = bf16_bits(dphi[ks][e] - bf16_val(dhi[e]));
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ph[ks][e] = pack2(hi[2 * e], hi[2 * e + 1]);
        pl[ks][e] = pack2(lo[2 * e], lo[2 * e + 1]);
        if (TAN) {
          dph[ks][e] = pack2(dhi[2 * e], dhi[2 * e + 1]);
          dpl[ks][e] = pack2(dlo[2 * e], dlo[2 * e + 1]);
        }
      }
    }
    const unsigned char* rec = a.comp + ((int64_t)bh * a.Mb + m) * kRec;
    const float* zc = reinterpret_cast<const float*>(rec + 32768);
    const float* dzc = reinterpret_cast<const float*>(rec + 33024);
    float dn = 0.f, ddn = 0.f;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 32 * ks + 8 * g + e;
        dn += phi[ks][e] * zc[d];
        if (TAN) ddn += dphi[ks][e] * zc[d] + phi[ks][e] * dzc[d];
      }
    dn = sum_over_groups(dn);
    dn = dn >= 0.f ? dn + a.eps_l : dn - a.eps_l;
    if (TAN) ddn = sum_over_groups(ddn);
    const float al = a.alpha[(int64_t)h * a.alpha_stride + m];
#pragma unroll
    for (int vt_ = 0; vt_ < 4; ++vt_) {
      f32x4 num = f32x4{0.f, 0.f, 0.f, 0.f}, dnum = num;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const unsigned char* hp = rec + ((vt_ * 2 + ks) * 64 + l) * 32;
        const u32x4 hh = *reinterpret_cast<const u32x4*>(hp);
        const u32x4 hl = *reinterpret_cast<const u32x4*>(hp + 16);
        num = mfma_bf16_16x16x32(hh, ph[ks], num);
        num = mfma_bf16_16x16x32(hh, pl[ks], num);
        num = mfma_bf16_16x16x32(hl, ph[ks], num);
        if (TAN) {
          const u32x4 dh = *reinterpret_cast<const u32x4*>(hp + 16384);
          const u32x4 dl = *reinterpret_cast<const u32x4*>(hp + 16384 + 16);
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
        const float ol = num[i] / dn;
        os[vt_][i] = al * os[vt_][i] + (1.f - al) * ol;
        if (TAN) {
          const float dol = (dnum[i] - ol * ddn) / dn;
          dos[vt_][i] = al * dos[vt_][i] + (1.f - al) * dol;
        }
      }
    }
  }

  if (qrow < L) {
    const int64_t oo = (qkbase + qrow) * kTa + 4 * g;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      *reinterpret_cast<f32x4*>(a.o + oo + 16 * ct) = os[ct];
      if (TAN) *reinterpret_cast<f32x4*>(a.dout + oo + 16 * ct) = dos[ct];
    }
  }
}

template <typename T16>
static void launch_fwd(const FwdArgs& a, bool tan, bool linear, int nblocks, hipStream_t st) {
  if (tan && linear)
    fwd_jvp_kernel<T16, true, true><<<nblocks, 256, 0, st>>>(a);
  else if (tan)
    fwd_jvp_kernel<T16, true, false><<<nblocks, 256, 0, st>>>(a);
  else if (linear)
    fwd_jvp_kernel<T16, false, true><<<nblocks, 256, 0, st>>>(a);
  else
    fwd_jvp_kernel<T16, false, false><<<nblocks, 256, 0, st>>>(a);
}

}  // namespace sla2h

using namespace sla2h;

extern "C" int sla2h_fwd_jvp(const void* q, const void* k, const void* dq, const void* dk,
                             const void* vt, const void* dvt, const int8_t* q8, const int8_t* k8,
                             const float* qs, const float* ks, const void* comp,
                             const float* alpha, int alpha_stride, const int32_t* lut, int dtype,
                             int B, int H, int64_t L, int D, int E, int Np, int T, float scale,
                             float eps_l, int flags, float* o, float* dout, void* stream) {
  SLA2H_CHECK_ARG(q && vt && q8 && k8 && qs && ks && lut && o);
  SLA2H_CHECK_ARG(D == kTa && E == kTa);
  SLA2H_CHECK_ARG(dtype == SLA2H_DTYPE_F16 || dtype == SLA2H_DTYPE_BF16);
  SLA2H_CHECK_ARG(B > 0 && H > 0 && L > 0 && Np > 0 && (int64_t)Np * E <= L);
  SLA2H_CHECK_ARG(T >= 1 && T <= Np);
  const bool tan = dq != nullptr;
  if (tan) SLA2H_CHECK_ARG(k && dk && dvt && dout);
  const bool linear = (flags & SLA2H_FLAG_SPARSE_ONLY) == 0;
  if (linear) SLA2H_CHECK_ARG(comp && alpha && alpha_stride >= 0);
  const int Nb = (int)((L + E - 1) / E);
  const int64_t nblocks = (int64_t)Nb * B * H;
  SLA2H_CHECK_ARG(nblocks < (1ll << 31));
  FwdArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.dq = static_cast<const uint16_t*>(dq);
  a.dk = static_cast<const uint16_t*>(dk);
  a.vt = static_cast<const uint16_t*>(vt);
  a.dvt = static_cast<const uint16_t*>(dvt);
  a.q8 = q8;
  a.k8 = k8;
  a.qs = qs;
  a.ks = ks;
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
  a.scale = scale;
  a.c_log2 = scale * 1.4426950408889634f;
  a.eps_l = eps_l;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == SLA2H_DTYPE_BF16)
    launch_fwd<BF16>(a, tan, linear, (int)nblocks, st);
  else
    launch_fwd<F16>(a, tan, linear, (int)nblocks, st);
  return (int)hipGetLastError();
}
