/*
 * sla2h.h -- C ABI of the MI355X (gfx950) SLA2 INT8 cube-attention hot path.
 *
 * Every entry point:
 *   - takes raw device pointers, sizes and a hipStream_t (passed as void*),
 *   - never allocates device memory (the caller owns inputs, outputs and the
 *     workspaces whose sizes the *_bytes() queries report),
 *   - is asynchronous on `stream` and re-entrant across streams,
 *   - returns 0 (hipSuccess) or a hipError_t code; 1 (hipErrorInvalidValue)
 *     for bad arguments.  sla2h_error_string() names a code.
 *
 * Tensor conventions (all contiguous, row-major):
 *   B batch, H heads, L tokens (tile-major order: Np video tiles of E tokens,
 *   then the P-token prefix as ceil(P/E) tail blocks), D head dim.
 *   E = D = 64 (one quantisation block = one attention tile = one MFMA tile).
 *   Nb = ceil(L/E) key/query blocks; Mb = Nb query blocks (LUT rows);
 *   n_tail = Nb - Np prefix tail blocks, always attended by the sparse branch.
 *   dtype: 0 = float16, 1 = bfloat16 (the 16-bit storage of q,k,v,dq,dk,dv).
 */
#ifndef SLA2H_H
#define SLA2H_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SLA2H_DTYPE_F16 0
#define SLA2H_DTYPE_BF16 1

/* sla2h_fwd_jvp flags */
#define SLA2H_FLAG_SPARSE_ONLY 1  /* write the sparse branch o_s only (no linear branch, no alpha mix) */

/* Library version and error names. */
int sla2h_version(void);
const char* sla2h_error_string(int code);

/*
 * Per-(b,h,E-token block) symmetric INT8 quantisation of one tensor,
 * E = 32, 64, 128 or 256.
 *   x  : (BH, L, D) 16-bit       -> xq (BH, L, D) int8,  xs (BH, ceil(L/E)) fp32
 *   s  = fl32(fl32(max|x|) / 127) + fl32(1e-12);  xq = round_half_away(x / s).
 * Replaces quantize_qkv / _quant_blocks
 * (models/sla2_vendor/kernel_sparse_qat.py:120-151).
 */
int sla2h_quantize(const void* x, int dtype, int64_t BH, int64_t L, int D, int E,
                   int8_t* xq, float* xs, void* stream);

/*
 * Fused INT8 quantisation of Q and K plus router tile pooling, one launch.
 *   q8,k8 (B,H,L,D) int8; qs,ks (B,H,Nb) fp32 (as sla2h_quantize);
 *   qpool (B,H,Nb,D) fp32: per-block mean of q over its real rows (sequential
 *     fp32 sum over rows, then / count), then optional projection
 *     qpool <- qpool @ proj_q^T (sequential fp32 dot, no FMA contraction);
 *   kpool_t (B,H,D,Np) fp32: the same for the Np video tiles of k, stored
 *     transposed (channel-major) for the router's coalesced score loop.
 *   proj_q / proj_k: (D,D) fp32 or NULL (identity).
 *   kbound (B,H,Nb) fp32 or NULL: per key block an upper bound on
 *     max_j ||k8_j|| * ks over its rows (sqrt of the largest fp32 row sum of
 *     squares of k, plus 4 ks for the int8 rounding), the input of the
 *     static softmax shift of sla2h_fwd_jvp.
 * Replaces the quantize_qkv(Q), quantize_qkv(K) calls of
 * sla2_cube_qat_jvp_fused (models/sla2_cube_qat.py:629-631) and the
 * _route_pool_kernel launches + projections of route_tiles_fast
 * (models/mla_video_sparse_jvp.py:506-562).
 */
int sla2h_quant_pool_qk(const void* q, const void* k, int dtype, int B, int H,
                        int64_t L, int D, int E, int Np,
                        const float* proj_q, const float* proj_k,
                        int8_t* q8, float* qs, int8_t* k8, float* ks,
                        float* qpool, float* kpool_t, float* kbound, void* stream);

/*
 * Block router: scores pc[m,n] = (sum_d qpool[m,d]*kpool[n,d]) * scale
 * (sequential fp32, no FMA), per row the T largest, ties to the lower index.
 *   lut (B,H,Mb,T) int32, each row ordered by descending score.
 *   mask (B,H,Mb,Np) uint8 or NULL: 1 where selected.
 * Np <= 4096.  Replaces the score GEMM + torch.topk of route_tiles_fast
 * (models/mla_video_sparse_jvp.py:563-565) and route_tiles (:292-294).
 */
int sla2h_route_topk(const float* qpool, const float* kpool_t, int B, int H,
                     int Mb, int Np, int D, int T, float scale,
                     int32_t* lut, uint8_t* mask, void* stream);

/*
 * Linear-branch states of the Np video tiles, phi = softmax over D:
 *   Hb  (B,H,Np,D,D) fp32 = phi(K_n)^T V_n
 *   dHb (B,H,Np,D,D) fp32 = dphi(K_n)^T V_n + phi(K_n)^T dV_n
 *   zb, dzb (B,H,Np,D) fp32 = column sums of phi(K_n), dphi(K_n)
 *   Hall,dHall (B,H,D,D), zall,dzall (B,H,D): sums over n (in n order);
 *     optional (NULL skips the summation).
 * Also writes the operand tiles of sla2h_fwd_jvp in MFMA fragment order (zero
 * past L; lane = 16 g + r, wave w = keys 16w..16w+15, column tile ct):
 *   vt (B,H,Nb,4,4,64,8) 16-bit with tangent: [ct][w][lane] = V[16w+4g+0..3][16ct+r]
 *      then dV of the same keys; (B,H,Nb,4,4,64,4) = V only without tangent;
 *   kt (B,H,Nb,4,4,64,8) 16-bit, tangent only: [w][ks][lane] = K[16w+r][32ks+8g+0..7]
 *      for ks 0,1 and dK[16w+r][32(ks-2)+8g+0..7] for ks 2,3.
 * dk, dv, dHb, dzb, dHall, dzall, kt may all be NULL (primal only).
 * Replaces _phi_states_kernel + the torch sums of sla2_cube_qat_jvp_fused
 * (models/sla2_cube_qat.py:634-648, 911-958).
 */
int sla2h_linear_states(const void* k, const void* dk, const void* v, const void* dv,
                        int dtype, int B, int H, int64_t L, int D, int E, int Np,
                        float* Hb, float* dHb, float* zb, float* dzb,
                        float* Hall, float* dHall, float* zall, float* dzall,
                        void* vt, void* kt, void* stream);

/* Bytes of one per-query-block complement record (see sla2h_complement). */
size_t sla2h_complement_record_bytes(int D);

/* Bytes of the workspace sla2h_complement needs (complement bit masks). */
size_t sla2h_complement_workspace_bytes(int B, int H, int Mb, int Np);

/*
 * Complement (non-routed video tiles) linear-branch states per query block:
 *   Hc[m] = sum_{n < Np, n not in lut[m,:]} Hb[n], and dHc, zc, dzc likewise,
 * computed per head as one 0/1-mask GEMM on bf16 MFMA (states split into
 * bf16 hi + lo, fp32 accumulate) and written as one record of
 * sla2h_complement_record_bytes(D) bytes per (b,h,m) in the operand layout
 * that sla2h_fwd_jvp consumes.  Tangent parts skipped when dHb == NULL.
 * workspace: sla2h_complement_workspace_bytes(B,H,Mb,Np) bytes.  Np <= 4096.
 * Replaces the in-loop complement-state subtraction of _cube_fused_jvp_kernel
 * (models/sla2_cube_qat.py:510-523, 570-578), which forms the same sums as
 * Hall - sum_{j<T} Hb[lut[m,j]].
 */
int sla2h_complement(const float* Hb, const float* dHb, const float* zb, const float* dzb,
                     const int32_t* lut, int B, int H, int Mb, int Np, int D, int T,
                     void* workspace, void* comp, void* stream);

/* Largest workspace sla2h_complement_noalloc serves (4 MiB: B*H up to 145 at
 * Mb = Np = 468, the 29,952-token shape). */
#define SLA2H_COMPLEMENT_SCRATCH_BYTES (4u << 20)

/*
 * sla2h_complement without the workspace argument: same kernels, same
 * records, bit for bit.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The bit-mask workspace is
 * a static device array of SLA2H_COMPLEMENT_SCRATCH_BYTES per GPU, held until
 * the process ends; calls whose sla2h_complement_workspace_bytes(B,H,Mb,Np)
 * exceeds it return hipErrorInvalidValue.  The call allocates nothing.  Every
 * call on one GPU shares that GPU's array (the current device's), so calls
 * that overlap on one GPU (other streams or threads) race.  The device
 * address of each GPU's array is looked up once, on the first call with that
 * device current.
 */
int sla2h_complement_noalloc(const float* Hb, const float* dHb, const float* zb,
                             const float* dzb, const int32_t* lut, int B, int H, int Mb,
                             int Np, int D, int T, void* comp, void* stream);

/*
 * The fused sparse + linear SLA2 op and its forward-mode JVP, tile-major:
 *   sparse branch: for each query block m, keys of tiles lut[m,0..T) and the
 *     n_tail prefix tail blocks; S = int32(q8 . k8^T) * (qs*ks); online softmax
 *     in exp2 with scale*log2(e); P.V on 16-bit MFMA;
 *     tangent: dS = (dq.k^T + q.dk^T)*scale, t = p*dS, do_s = (t.V + p.dV)/l
 *     - (mu/l) o_s (t saturated at +-60000 for fp16 operands);
 *   linear branch: o_l = phi(q) Hc / den, den = phi(q).zc (+-eps_l, signed);
 *     do_l by the quotient rule; o = a o_s + (1-a) o_l, a = alpha[h*alpha_stride+m].
 *   Outputs o, dout (B,H,L,D) fp32.  Tangent inputs/outputs NULL = primal only.
 *   vt, kt = the operand tiles of sla2h_linear_states (tangent layouts and kt
 *   required when dq is given).
 *   comp = sla2h_complement records (unused with SLA2H_FLAG_SPARSE_ONLY).
 *   kb = the kbound output of sla2h_quant_pool_qk, or NULL.  Given kb, a query
 *     block whose score factors qs*ks*scale*log2(e) stay <= 2^-9 runs with a
 *     fixed per-row softmax shift (a Cauchy-Schwarz bound on the row's
 *     scores) instead of a running maximum, and falls back to the running
 *     maximum when a row's sum lands below 2^-64; the softmax is the same up
 *     to fp32 and 16-bit rounding.
 * Replaces _cube_fused_jvp_kernel (models/sla2_cube_qat.py:448-602) and,
 * with SLA2H_FLAG_SPARSE_ONLY, _sla2_cube_jvp_qat_kernel's sparse branch
 * (models/sla2_cube_qat.py:59-169, 172-207).
 */
int sla2h_fwd_jvp(const void* q, const void* dq, const void* kt, const void* vt,
                  const int8_t* q8, const int8_t* k8,
                  const float* qs, const float* ks, const float* kb, const void* comp,
                  const float* alpha, int alpha_stride, const int32_t* lut,
                  int dtype, int B, int H, int64_t L, int D, int E, int Np, int T,
                  float scale, float eps_l, int flags,
                  float* o, float* dout, void* stream);

/* ---- 1-D SLA2 blocks (query blocks of bq rows, key blocks of 64) -------- */

/*
 * Block means for the 1-D router: out[bh][j][d] (or [bh][d][j] when
 * transposed) = sum over the real rows t of block j (blk rows, the last block
 * ragged) of x[bh][t][d] / count, sequential fp32 in row order; then, when
 * proj (D,D) fp32 is given, out[e] = sum_d mean[d] proj[e][d] (sequential, no
 * contraction).  Replaces _block_pool + projections of route_blocks
 * (models/sla2_mla_jvp.py:51-99) and mean_pool_smooth + proj_q/proj_k of the
 * SLA2 Router (models/sla2_vendor/kernel_router.py:373-404,
 * models/sla2_vendor/router.py:66-75); the smooth-k shift is a per-row
 * constant of the scores and leaves the top-k selection unchanged.
 * Feed the pooled queries and the transposed pooled keys to sla2h_route_topk
 * with Mb = ceil(L/bq) and Np = ceil(L/64).  dtype: SLA2H_DTYPE_F16,
 * SLA2H_DTYPE_BF16 or 2 (fp32 input, pooled as given: the reference's router
 * reads q and k in their own dtype).
 */
int sla2h_pool_blocks(const void* x, int dtype, int64_t BH, int64_t L, int D, int blk,
                      const float* proj, int transposed, float* out, void* stream);

/*
 * 1-D SLA2 attention with forward-mode JVP (sla2_mla_jvp): as sla2h_fwd_jvp but
 * with 16-bit primal scores S = q.k^T (fp32 accumulate; no INT8), query blocks
 * of bq rows (bq = 64, 128 or 256; lut (B,H,ceil(L/bq),T), alpha (H,
 * ceil(L/bq)) and comp records per query block), every key block routable
 * (Np = Nb, the last one partial when 64 does not divide L) and no prefix
 * tail.  kt, vt from sla2h_linear_states(Np = Nb) with tangents; comp from
 * sla2h_complement(Mb = ceil(L/bq), Np = Nb).  Tangents are required.
 * Replaces _sla2_sparse_jvp_kernel + _linear_jvp + the mix of sla2_mla_jvp
 * (models/sla2_mla_jvp.py:108-237, 258-342, 348-385).
 */
int sla2h_fwd_jvp_1d(const void* q, const void* dq, const void* kt, const void* vt,
                     const void* comp, const float* alpha, int alpha_stride, const int32_t* lut,
                     int dtype, int B, int H, int64_t L, int D, int bq, int bk, int T,
                     float scale, float eps_l, float* o, float* dout, void* stream);

/* ---- MLA sublayer / MLP sublayer JVP stages (row kernels) --------------- */

/*
 * RMSNorm JVP over rows of width D (<= 1024): y = w x / r,
 * dy = w (dx / r - x mean(x dx) / r^3), r = sqrt(mean(x^2) + eps), fp32 math.
 * x, dx rows at stride sx; y, dy rows at stride sy (elements).  in_dtype /
 * out_dtype: SLA2H_DTYPE_F16, SLA2H_DTYPE_BF16 or 2 (fp32); fp32 -> 16-bit,
 * fp32 -> fp32 and 16-bit -> same 16-bit are supported.  Replaces
 * _rmsnorm_jvp_strided (models/triton_mla_block_jvp.py:237-268).
 */
int sla2h_rmsnorm_jvp(const void* x, const void* dx, int in_dtype, const float* w, int64_t rows,
                      int D, int64_t sx, void* y, void* dy, int64_t sy, int out_dtype, float eps,
                      void* stream);

/*
 * MLA head preparation from the stacked [primal; tangent] GEMM outputs
 * (2*B*S rows): qb (2BS, H*(dn+dr)) = per head [q_nope | q_rope];
 * kvb (2BS, H*(dn+dv)) = per head [k_nope | v]; kr = the shared k_rope band
 * (dr values at row stride skr, e.g. a column slice of the fused q_a/kv_a
 * output).  Per head: RMSNorm JVP of the nope bands (w_qnorm / w_knorm, dn),
 * RoPE rotation of (2i, 2i+1) pairs by rope_cos/sin (S, dr/2) fp32, v copied.
 * Outputs q, dq, k, dk, v, dv as (B, H, L=S, 64) 16-bit, token s written at row
 * pos[s] (pos (S,) int32, e.g. the inverse tile permutation) or s when pos is
 * NULL.  dn = dr = 32, dv = 64.  Replaces _q_prep_kernel / _kv_prep_kernel and
 * the (B,S,H,hd) -> (B,H,L,hd) [perm] copies (models/triton_mla_block_jvp.py:
 * 279-425, models/mla_jvp_fast.py:95-136).
 */
int sla2h_mla_qkv_prep(const void* qb, const void* kvb, const void* kr, int64_t skr,
                       const float* w_qnorm, const float* w_knorm, const float* rope_cos,
                       const float* rope_sin, const int32_t* pos, int dtype, int B, int S, int H,
                       int dn, int dr, int dv, float eps, void* q, void* dq, void* k, void* dk,
                       void* v, void* dv_out, void* stream);

/*
 * Attention output back to model order, rounded to 16 bits, and the output
 * gate's JVP: out (2BS, H*dv) stacked, primal row (b,s) = a sigmoid(z), tangent
 * row = da sigmoid(z) + a sigmoid(z)(1 - sigmoid(z)) dz, with a, da the op's
 * (B,H,L,dv) fp32 outputs at row pos[s] (or s) and z (2BS, H*dv) 16-bit
 * stacked gate logits; z NULL = no gate.  Replaces the attention-buffer
 * scatter and _out_gate_jvp_kernel (models/mla_jvp_fast.py:142-193,
 * models/triton_mla_block_jvp.py:480-498).
 */
int sla2h_mla_out_gate(const float* o, const float* dout, const int32_t* pos, const void* z,
                       int dtype, int B, int S, int H, int dv, void* out, void* stream);

/*
 * SituAndMul JVP on stacked rows: gu (2*rows, 2F) = [gate | up] per row,
 * primal rows first; act (2*rows, F): h = situ(g) u, dh = situ'(g) dg u +
 * situ(g) du, situ(g) = beta tanh(g / beta) sigmoid(g).  Replaces
 * _swiglu_row_jvp (models/triton_mla_block_jvp.py:437-471).
 */
int sla2h_situ_jvp(const void* gu, int64_t rows, int F, float beta, int dtype, void* act,
                   void* stream);

/*
 * SituAndMul of the DiT block's training forward and its backward (the
 * autograd path): h = situ(g) u', situ(g) = beta tanh(g / beta) sigmoid(g),
 * u' = lb tanh(u / lb) for lb > 0 (the linear_beta soft clamp), else u;
 * dg = dh u' situ'(g), du = dh situ(g) du'/du.  gate / up: (rows, F) with row
 * strides sg / su elements (views of one [gate | up] tensor allowed); out, dh,
 * dgate, dup: contiguous (rows, F).  dtype: SLA2H_DTYPE_F16, SLA2H_DTYPE_BF16
 * or 2 (fp32); fp32 arithmetic.  16-byte accesses when F, the strides and the
 * pointers allow them (multiples of 8 elements for 16-bit, 4 for fp32), else
 * one element per thread.
 * Replaces the eager SituAndMul.forward and its autograd backward
 * (models/imf_dit_video.py:136-171).
 */
int sla2h_situ_mul_fwd(const void* gate, const void* up, int dtype, int64_t rows, int F,
                       int64_t sg, int64_t su, float beta, float lb, void* out, void* stream);
int sla2h_situ_mul_bwd(const void* dh, const void* gate, const void* up, int dtype, int64_t rows,
                       int F, int64_t sg, int64_t su, float beta, float lb, void* dgate,
                       void* dup, void* stream);

/*
 * RMSNorm of the DiT block's training forward and its backward (the autograd
 * path): y = round_x(x r) w, r = 1 / sqrt(mean(x^2) + eps) in fp32, round_x the
 * rounding to x's dtype, w fp32, y fp32 contiguous (rows, D).  Backward:
 * g = round_x(dy w), dx = round_x(r g - x r^3 mean(g x)) contiguous in x's
 * dtype, dw = sum over rows of round_x(x r) dy (deterministic two-step sum in
 * `workspace` of sla2h_rmsnorm_bwd_workspace_bytes).  x: (rows, D <= 1024),
 * row stride sx elements; dtype SLA2H_DTYPE_F16, SLA2H_DTYPE_BF16 or 2 (fp32).
 * Replaces RMSNorm.forward and its autograd backward
 * (models/imf_dit_video.py:121-133).
 */
int sla2h_rmsnorm_fwd(const void* x, int dtype, int64_t rows, int D, int64_t sx, const float* w,
                      float eps, float* y, void* stream);
size_t sla2h_rmsnorm_bwd_workspace_bytes(int64_t rows, int D);
int sla2h_rmsnorm_bwd(const void* x, int dtype, int64_t rows, int D, int64_t sx, const float* w,
                      const float* dy, float eps, void* dx, float* dw, void* workspace,
                      void* stream);

/*
 * The same RMSNorm for an fp32 residual stream feeding 16-bit consumers (the
 * block's linears under autocast): y16 = round16(x r w) in out_dtype, the
 * fp32 output of sla2h_rmsnorm_fwd rounded once (what the consumers' casts
 * would produce), contiguous (rows, D).  Backward: the output gradient is
 * dy0 + dy1 + dy2 (16-bit, dy1 / dy2 may be NULL), summed in fp32 in that
 * order (the consumers' gradients, each cast to fp32 as autocast's cast
 * backward does), then sla2h_rmsnorm_bwd's math, plus dadd (fp32 or NULL:
 * the gradient x receives from its other use, the residual add) added to dx
 * (fp32).  D a power of two <= 512; every pointer 16-byte aligned; workspace
 * of sla2h_rmsnorm_bwd_workspace_bytes.  Replaces RMSNorm.forward
 * (models/imf_dit_video.py:129-133) at norm1 / norm2 of TransformerBlock.forward
 * (:529-532) under torch.autocast, the casts of its output at the linears that
 * read it (:436, :440, :466; :187) and the fp32 gradient accumulations of the
 * backward.
 */
/*
 * The MLA sublayer's output gate on 16-bit tensors (autocast), n elements
 * (n % 8 == 0, 16-byte aligned, same dtype):
 *   s = round16(1 / (1 + exp(-g))), out = round16(a s);
 *   backward: da = round16(dout s),
 *   dg = round16(round16(round16(dout a) round16(1 - s)) s),
 * the rounding points of torch's GPU sigmoid, mul and their backward (the
 * sigmoid backward works in the 16-bit type, one rounding per operation).  Replaces
 * attn * torch.sigmoid(self.g_proj(x)) (models/imf_dit_video.py:466).
 */
int sla2h_gate_mul_fwd(const void* a, const void* g, int dtype, int64_t n, void* out,
                       void* stream);
int sla2h_gate_mul_bwd(const void* dout, const void* a, const void* g, int dtype, int64_t n,
                       void* da, void* dg, void* stream);

/*
 * The MLA sublayer's attention operands for a tile-major SLA2 op: replaces
 * q = torch.cat([q_nope, q_rope], -1), k = torch.cat([k_nope, k_rope], -1)
 * and the op's permute(0, 2, 1, 3).half() of q, k, v
 * (models/imf_dit_video.py:458-463, models/sla2_cube_qat.py:340-350).
 * An operand is two 32-channel halves, each addressed by element strides
 * (sb, st, sh) over (batch, token, head); sh = 0 for a half the heads share
 * (the key's rope band).  lo_dtype: SLA2H_DTYPE_F16, SLA2H_DTYPE_BF16 or 2
 * (fp32, the per-head RMSNorm output); hi_dtype 16-bit.  Bases and strides
 * 16-byte multiples.  out: (B, H, L, 64) fp16, every value converted once.
 * Backward: dout (B, H, L, 64) fp16 -> each half's gradient in the half's
 * dtype at its strides (exact for fp32, one rounding for 16-bit); with
 * hi_sh = 0 the shared half gets the fp32 sum over the heads, in head order,
 * of the per-head 16-bit gradients, rounded once.
 */
int sla2h_attn_in_fwd(const void* lo, int lo_dtype, int64_t lo_sb, int64_t lo_st, int64_t lo_sh,
                      const void* hi, int hi_dtype, int64_t hi_sb, int64_t hi_st, int64_t hi_sh,
                      int B, int H, int64_t L, void* out, void* stream);
int sla2h_attn_in_bwd(const void* dout, void* dlo, int lo_dtype, int64_t lo_sb, int64_t lo_st,
                      int64_t lo_sh, void* dhi, int hi_dtype, int64_t hi_sb, int64_t hi_st,
                      int64_t hi_sh, int B, int H, int64_t L, void* stream);

/*
 * The output gate after a tile-major SLA2 op under autocast: replaces
 * o.permute(0, 2, 1, 3).to(float32) (models/sla2_cube_qat.py:397-400), the
 * gate attn * torch.sigmoid(g) in fp32 (models/imf_dit_video.py:466) and the
 * output projection's autocast cast of its input.  o: (B, H, L, 64) fp16;
 * g, out: (B, L, H * 64) in dtype (16-bit, the autocast dtype):
 *   s = round16(sigmoid(g)), out = round16(fp32(o) s);
 *   backward from dy (B, L, H * 64) in dtype: do = fp16(dy s) in o's layout,
 *   dg = round16(round16(round16(dy fp32(o)) round16(1 - s)) s).
 */
int sla2h_attn_gate_fwd(const void* o, const void* g, int dtype, int B, int H, int64_t L,
                        void* out, void* stream);
int sla2h_attn_gate_bwd(const void* dy, const void* o, const void* g, int dtype, int B, int H,
                        int64_t L, void* dout, void* dg, void* stream);

int sla2h_rmsnorm_fwd16(const float* x, int64_t rows, int D, int64_t sx, const float* w,
                        float eps, int out_dtype, void* y, void* stream);
int sla2h_rmsnorm_bwd_sum(const float* x, int64_t rows, int D, int64_t sx, const float* w,
                          const void* dy0, const void* dy1, const void* dy2, int dy_dtype,
                          const float* dadd, float eps, float* dx, float* dw, void* workspace,
                          void* stream);

/*
 * RoPE of the DiT block's training forward and its backward: channel pairs
 * (2i, 2i+1) of x (B, L, H, hd), strides sb / sl / sh elements and unit
 * channel stride, rotated by the angles of token l (cos_t / sin_t (L, hd/2)
 * fp32) in fp32 and written contiguous (B, L, H, hd) in x's dtype; inverse = 1
 * rotates by the negated angles (the backward of the output gradient).
 * Replaces apply_rotary_pos_emb and its autograd backward
 * (models/imf_dit_video.py:266-284).
 */
int sla2h_rope(const void* x, int dtype, int64_t B, int64_t L, int H, int hd, int64_t sb,
               int64_t sl, int64_t sh, const float* cos_t, const float* sin_t, int inverse,
               void* out, void* stream);

/*
 * ReZero residual of the DiT block's training forward and its backward:
 * y = x + a s (x, y fp32 (rows, D) contiguous; a (rows, D) contiguous in
 * dtype SLA2H_DTYPE_F16 / SLA2H_DTYPE_BF16 / 2 (fp32); s fp32 (D)), product and
 * sum rounded separately.  Backward: da = round_a(dy s), ds = sum over rows of
 * dy a (deterministic two-step sum in `workspace` of
 * sla2h_residual_scale_bwd_workspace_bytes).  Replaces `x + sublayer(x) * scale`
 * and its autograd backward (models/imf_dit_video.py:529-532).
 */
int sla2h_residual_scale_fwd(const float* x, const void* a, int dtype, const float* s,
                             int64_t rows, int D, float* y, void* stream);
size_t sla2h_residual_scale_bwd_workspace_bytes(int64_t rows, int D);
int sla2h_residual_scale_bwd(const float* dy, const void* a, int dtype, const float* s,
                             int64_t rows, int D, void* da, float* ds, void* workspace,
                             void* stream);

/* ---- training forward (the module's autograd forward) ------------------ */

/*
 * Per-(b,h,64-token block) INT8 quantisation of Q, K and V with the
 * training kernel's law: s = fl32(max|x| / 127) + 1e-12,
 * x8 = trunc(fl32(fl32(x / s) + 0.5 sign(x))) (toward zero; sign(+-0) = +1).
 *   q8,k8 (B,H,L,D) int8; qs,ks,vs (B,H,Nb) fp32;
 *   v8f (B,H,Nb,4,64,16) int8, the value tile in INT8 MFMA fragment order:
 *     [ct][lane][s] = V8[16(s>>2) + 4g + (s&3)][16ct + r], lane = 16g + r,
 *     rows past L zero.
 * 3*B*H <= 65535.  Replaces the in-kernel quantisation of _attn_fwd_qat
 * (models/sla2_vendor/kernel_sparse_qat.py:56-58, 88-90, 106-107).
 */
int sla2h_quant_train(const void* q, const void* k, const void* v, int dtype, int B, int H,
                      int64_t L, int D, int E, int8_t* q8, float* qs, int8_t* k8, float* ks,
                      int8_t* v8f, float* vs, void* stream);

/*
 * Sparse branch of the training forward over the augmented LUT (lut[m,0..T)
 * then the Nb-Np prefix tail blocks):
 *   S = int32(q8 . k8^T) * (qs*ks) * fl32(scale*log2 e), keys past L masked;
 *   exact running max per 64-key tile, P = exp2(S - m),
 *   P8 = (int) fl(127 P + 0.5), O += int32(P8 . V8) * (vs/127);
 *   o_s = O / l (B,H,L,D) 16-bit, lse = m + log2 l (B,H,L) fp32 (log2 domain),
 *   qphi = softmax_D(q) (B,H,L,D) 16-bit.
 * Inputs from sla2h_quant_train.  T + (Nb - Np) <= 1024.  Replaces
 * _attn_fwd_qat with USE_INT8 and PHI_OUT
 * (models/sla2_vendor/kernel_sparse_qat.py:28-117) as launched by
 * _CubeQATFunction.forward (models/sla2_cube_qat.py:717-722).
 */
int sla2h_sparse_fwd_qat(const void* q, const int8_t* q8, const float* qs, const int8_t* k8,
                         const float* ks, const int8_t* v8f, const float* vs,
                         const int32_t* lut, int dtype, int B, int H, int64_t L, int D, int E,
                         int Np, int T, float scale, void* o_s, float* lse, void* qphi,
                         void* stream);

/*
 * Linear-branch states of ALL Nb tiles with phi(K) rounded to the 16-bit type
 * first (softmax(K).to(dtype)), rows past L zero:
 *   Hb (B,H,Nb,D,D), zb (B,H,Nb,D) fp32 per tile; Hall (B,H,D,D), zall (B,H,D)
 *   fp32 sums over the tiles in n order (= htot and ztot before rounding).
 * Feed Hb/zb to sla2h_complement with Np = Nb and the augmented LUT.
 * vt (B,H,Nb,4,4,64,4) 16-bit or NULL: the primal value operand tiles (as
 * sla2h_linear_states writes them), needed by sla2h_sparse_fwd_1d.
 * Replaces kphi = softmax(kh).to(dtype) and _precompute_global
 * (models/sla2_cube_qat.py:728-730; models/sla2_vendor/kernel_linear.py:305-313).
 */
int sla2h_linear_states_qat(const void* k, const void* v, int dtype, int B, int H, int64_t L,
                            int D, int E, float* Hb, float* zb, float* Hall, float* zall,
                            void* vt, void* stream);

/*
 * Linear branch (state form) and alpha mix of the training forward:
 *   H_m = round16(comp.Hc[m] + (round16(Hall) - Hall)), z_m = comp.zc[m];
 *   den = qphi . z_m (+-eps_l, signed) (B,H,L) fp32;
 *   o_l = round16(qphi H_m / den) (B,H,L,D) 16-bit;
 *   o = round16(round16(a o_s) + round16(round16(1 - a) o_l)), a =
 *   round16(alpha[h*alpha_stride + m]) (B,H,L,D) 16-bit.
 * comp = sla2h_complement records over the augmented LUT.  E = the query block
 * length (64 for the cube; 64, 128 or 256 for 1-D blocks): records and alpha
 * are per query block of E rows.  Replaces _lin_fwd2
 * without SCORE_FORM (models/sla2_vendor/kernel_linear.py:206-304) and the mix
 * of _CubeQATFunction.forward (models/sla2_cube_qat.py:733-744).
 */
int sla2h_linear_mix_qat(const void* qphi, const void* comp, const float* Hall,
                         const void* o_s, const float* alpha, int alpha_stride, int dtype,
                         int B, int H, int64_t L, int D, int E, float eps_l, void* o,
                         void* o_l, float* den, void* stream);

/*
 * Score form of the same linear branch and mix, which the reference runs while
 * the augmented LUT has at most 4 columns (T + n_tail <= 4):
 *   W_j = qphi kphi_j^T (fp32), kphi_j = round16(softmax_D(k rows of tile j)),
 *     rows past L zero;
 *   num = qphi round16(Hall) - sum_j round16(W_j) v_j (fp32 accumulate);
 *   den = qphi . zall - sum_j rowsum(W_j), then +-eps_l (signed);
 *   o_l, o and den as sla2h_linear_mix_qat.
 * k, v (B,H,L,D) 16-bit; Hall (B,H,D,D), zall (B,H,D) fp32 from
 * sla2h_linear_states_qat; lut (B,H,ceil(L/E),J) int32, ids in [0, ceil(L/64))
 * (ids outside are clamped; the Python layer rejects them), J <= 1024.
 * Replaces _lin_fwd2 with SCORE_FORM (models/sla2_vendor/kernel_linear.py:
 * 206-272) as selected at models/sla2_cube_qat.py:424, 739 and
 * models/sla2_vendor/kernel_linear.py:357.
 */
int sla2h_linear_mix_score(const void* qphi, const void* k, const void* v, const float* Hall,
                           const float* zall, const int32_t* lut, int J, const void* o_s,
                           const float* alpha, int alpha_stride, int dtype, int B, int H,
                           int64_t L, int D, int E, float eps_l, void* o, void* o_l, float* den,
                           void* stream);

/*
 * Workspace of sla2h_sla2_forward_fused in bytes (0 for invalid sizes).
 */
size_t sla2h_sla2_fused_workspace_bytes(int B, int H, int64_t L, int D);

/*
 * Fused SLA2 inference forward with the arithmetic of the fused Algorithm-2
 * kernel, for the 1-D module with fused=True:
 *   sparse branch: INT8 (q8 != NULL; Q scales qs per block_m rows from
 *     sla2h_quantize, K8, V8 as for sla2h_sparse_fwd_int8) or 16-bit (q8 ==
 *     NULL; vt the value operand tiles of sla2h_linear_states_qat), o_s = O / l
 *     kept in fp32;
 *   linear branch: the score form of sla2h_linear_mix_score against
 *     round16(Hall), zall (sla2h_linear_states_qat over the whole sequence);
 *   o = round16(a o_s + (1 - a) num / den) in fp32, a = alpha[h*alpha_stride + m]
 *     unrounded (the reference averages alpha over heads for this kernel: pass
 *     alpha_stride 0 with the averaged row).
 * lut (B,H,ceil(L/bq),T) int32 key blocks of 64 rows; workspace of
 * sla2h_sla2_fused_workspace_bytes(B,H,L,D) bytes.  Two launches on stream.
 * Replaces sla2_forward_fused / _sla2_fwd_fused
 * (models/sla2_vendor/kernel_fused.py:29-160) as called at
 * models/sla2_vendor/core.py:93-106.
 */
int sla2h_sla2_forward_fused(const void* q, const void* k, const void* v, const int8_t* q8,
                             const float* qs, int block_m, const int8_t* k8, const float* ks,
                             const int8_t* v8f, const float* vs, const void* vt,
                             const float* Hall, const float* zall, const int32_t* lut, int T,
                             const float* alpha, int alpha_stride, int dtype, int B, int H,
                             int64_t L, int D, int bq, float scale, float eps_l, void* workspace,
                             void* o, void* stream);

/*
 * 16-bit sparse branch of the 1-D training forward (no INT8): S = q.k^T on
 * 16-bit MFMA (fp32 accumulate) * scale * log2(e) over the routed key blocks
 * of each query block of bq rows (lut (B,H,ceil(L/bq),T)), exact running
 * maximum, O += round16(P).V; o_s = O / l (16-bit), lse = m + log2 l (fp32),
 * qphi = softmax_D(q) (16-bit).  vt from sla2h_linear_states_qat.  Replaces
 * _attn_fwd_qat without USE_INT8 (models/sla2_vendor/kernel_sparse_qat.py:28-117)
 * as run by _sparse_attention_qat (:265-293) for the SLA2 module.
 */
int sla2h_sparse_fwd_1d(const void* q, const void* k, const void* vt, const int32_t* lut,
                        int dtype, int B, int H, int64_t L, int D, int bq, int bk, int T,
                        float scale, void* o_s, float* lse, void* qphi, void* stream);

/* ---- training backward (straight-through estimator) --------------------- */

/*
 * Per 64-row block: the gradient split and the row statistics of the
 * backward.
 *   dos = round16(fl32(dout * a)), do_l = round16(fl32(dout * (1 - a))),
 *     a = alpha[h,m] fp32 (the fp32 product rounds first, as in the reference);
 *   delta = sum_d o_s * dos (B,H,L) fp32;
 *   g16 = round16(sat(do_l / den)) (B,H,L,D) 16-bit, s = sum_d do_l o_l / den (B,H,L);
 *   seg (H,Mb) fp32 += sum over the block of dout * (o_s - o_l) (atomic over b;
 *     zero it first), so d(alpha logit) = seg * a * (1 - a);
 *   P = qphi^T sat(g) (B,H,Mb,D,D) fp32, Pz = qphi^T s (B,H,Mb,D) fp32.
 * sat(x) = clamp(x, -60000, 60000).  E = the query block length (64, or 128 /
 * 256 for 1-D blocks): alpha and seg have one column per query block of E
 * rows; every other array is per 64-row block.  Replaces _bwd_split_kernel
 * (models/sla2_cube_qat.py:838-872), _attn_bwd_preprocess
 * (models/sla2_vendor/sla_kernel.py:89-114) and the g, s, dhtot, dztot torch
 * lines of _CubeQATFunction.backward (models/sla2_cube_qat.py:765-797).
 */
int sla2h_bwd_prep(const void* dout, const void* o_s, const void* o_l, const float* den,
                   const void* qphi, const float* alpha, int alpha_stride, int dtype, int B,
                   int H, int64_t L, int D, int E, void* dos, float* delta, void* g16, float* s,
                   float* seg, float* P, float* Pz, void* stream);

/*
 * Backward complement over the augmented LUT lut_aug (B,H,ceil(Mb*64/bq),J) int32,
 * one row per query block of bq rows (bq = 64 for the cube), Mb 64-row blocks:
 *   sel (B,H,Mb,ceil(Mb/32)) uint32: bit j of word kc of tile n = 1 where query
 *     block 32kc + j routes tile n;
 *   comp records (B,H,Mb, sla2h_complement_record_bytes(64) bytes), fp32:
 *     Hc[n] = sum_{m not routing n} P[m] (the complement dh), zc[n] = sum Pz[m].
 * workspace: sla2h_complement_workspace_bytes(B,H,Mb,Mb) bytes.  Mb <= 4096
 * (query blocks = key tiles).  Replaces _invert_lut and the dhtot/dztot minus
 * selected-blocks loop of _lin_bwd_dkdv_lut (models/sla2_cube_qat.py:966-983,
 * 1045-1095).
 */
int sla2h_complement_bwd(const float* P, const float* Pz, const int32_t* lut_aug, int B, int H,
                         int Mb, int bq, int J, void* workspace, uint32_t* sel, void* comp,
                         void* stream);

/*
 * dq = round16(sat(dq_s + qphi (dqphi - <qphi, dqphi>))) (B,H,L,D) 16-bit, with
 *   dq_s = round16(scale sum_tiles round16(sat(p (dos.v - delta))) k),
 *   p = exp2(min(q.k scale log2e - lse, 4)) on the unquantised 16-bit q, k;
 *   dqphi = g16 H16^T - s z^T, H16 = round16(comp.Hc + (round16(Hall) - Hall)),
 *   z = comp.zc (comp, Hall, lse, qphi from the training forward).
 * J = columns of lut_aug <= 1024; E = the query block length (LUT rows and comp
 * records per query block of E rows).  Replaces _attn_bwd_dq
 * (models/sla2_vendor/sla_kernel.py:117-184), _lin_bwd_dq
 * (models/sla2_vendor/kernel_linear.py:85-138) and the Q-side
 * _phi_chain_add_kernel (models/sla2_cube_qat.py:875-904, 814-818).
 */
int sla2h_bwd_dq(const void* q, const void* k, const void* v, const void* dos, const float* lse,
                 const float* delta, const void* g16, const float* s, const void* comp,
                 const float* Hall, const void* qphi, const int32_t* lut_aug, int dtype, int B,
                 int H, int64_t L, int D, int E, int J, float scale, void* dq, void* stream);

/*
 * dk = round16(sat(dk_s + kphi (dkphi - <kphi, dkphi>))), dv = round16(sat(dv_s + dv_l))
 * (B,H,L,D) 16-bit, over the query blocks that route each key tile (sel):
 *   dk_s = round16(scale sum round16(sat(p (dos.v - delta)))^T q),
 *   dv_s = round16(sum round16(p)^T dos);
 *   dkphi = v dh16^T + dz, dv_l = kphi dh16, dh16 = round16(sat(comp_bwd.Hc)),
 *   dz = -comp_bwd.zc, kphi = round16(softmax_D(k)).
 * Replaces _sparse_bwd_dkdv_lut (models/sla2_cube_qat.py:986-1042),
 * _lin_bwd_dkdv_lut (:1045-1104), the K-side _phi_chain_add_kernel and the dv
 * sum (:819-830).
 */
int sla2h_bwd_dkdv(const void* q, const void* k, const void* v, const void* dos, const float* lse,
                   const float* delta, const uint32_t* sel, const void* comp_bwd, int dtype,
                   int B, int H, int64_t L, int D, int E, float scale, void* dk, void* dv,
                   void* stream);

/* ---------------------------------------------------------------------
 * Inference path of the 1-D SLA2 module (no-grad forward).
 * --------------------------------------------------------------------- */

/*
 * The training forward's truncating INT8 law (sla2h_quant_train's) for one
 * tensor in blocks of E = 32, 64, 128 or 256 rows:
 *   s = fl32(fl32(max|x|) / 127) + fl32(1e-12);  xq = (int) fl(fl(x / s) + 0.5 sign(x)).
 * Q of the 1-D SLA2 INT8 training forward (query tiles of bq rows); replaces
 * the in-kernel Q quantisation of _attn_fwd_qat with USE_INT8
 * (models/sla2_vendor/kernel_sparse_qat.py:56-58).
 */
int sla2h_quantize_trunc(const void* x, int dtype, int64_t BH, int64_t L, int D, int E,
                         int8_t* xq, float* xs, void* stream);

/*
 * V of the inference INT8 path: sla2h_quantize's law (E = 64) written in the
 * INT8 MFMA fragment order of sla2h_quant_train's v8f (BH, Nb, 4096).
 * Replaces quantize_qkv(v, BLOCK_N) as sparse_attention_int8 calls it
 * (models/sla2_vendor/kernel_sparse_qat.py:238-239).
 */
int sla2h_quantize_v8f(const void* v, int dtype, int64_t BH, int64_t L, int D, int E,
                       int8_t* v8f, float* vs, void* stream);

/*
 * Inference INT8 sparse branch, every key block routable (the last one may be
 * partial), query blocks of bq = 64/128/256 rows for the LUT (B,H,ceil(L/bq),T):
 *   S = int32(Q8 . K8^T) * (sq * sk) * scale * log2(e), keys past L masked,
 *   exact running maximum, P8 = (int) fl(127 P + 0.5), O += int32(P8 . V8) * sv/127,
 *   o_s = O / l (16-bit), lse = m + log2(l), qphi = softmax_D(q) (16-bit, optional).
 * q8/qs from sla2h_quantize with E = qblock (32..256; bq for the unfused path,
 * block_m for the fused one), k8/ks from sla2h_quantize (E = 64), v8f/vs from
 * sla2h_quantize_v8f.  Replaces _attn_fwd_int8 / sparse_attention_int8
 * (models/sla2_vendor/kernel_sparse_qat.py:154-247) and the INT8 sparse half of
 * _sla2_fwd_fused (models/sla2_vendor/kernel_fused.py:81-106).
 */
int sla2h_sparse_fwd_int8(const void* q, const int8_t* q8, const float* qs, int qblock,
                          const int8_t* k8, const float* ks, const int8_t* v8f, const float* vs,
                          const int32_t* lut, int dtype, int B, int H, int64_t L, int D, int bq,
                          int T, float scale, void* o_s, float* lse, void* qphi, void* stream);

/*
 * Inference linear-branch states of every 64-row key block:
 *   Hb[j] = round16(round16(phi(K_j))^T V_j) (held as fp32 values, fp32 accumulate),
 *   zb[j] = colsum round16(phi(K_j)) (fp32), phi = softmax over D;
 *   Hall / zall = the sums over the blocks when given (both or neither);
 *   vt (optional): the primal value operand tiles of sla2h_linear_states.
 * Replaces _hblocks and the totals of complement_linear_states
 * (models/sla2_vendor/kernel_linear.py:396-427, 496-504).
 */
int sla2h_hblocks_states(const void* k, const void* v, int dtype, int B, int H, int64_t L, int D,
                         int E, float* Hb, float* zb, float* Hall, float* zall, void* vt,
                         void* stream);

/*
 * Linear branch and mix of the inference path, per query row of block i
 * (bq = 64/128/256 rows):
 *   H_i = round16(comp.Hc), num = qphi . H_i (fp32 accumulate), den = qphi . comp.zc,
 *   den += eps_l signed, o_l = num / den, o = round16(a o_s + (1 - a) o_l),
 *   a = alpha[h * alpha_stride + i] (fp32).
 * comp: sla2h_complement records over the plain LUT of sla2h_hblocks_states.
 * Replaces _lin_fwd3 (models/sla2_vendor/kernel_linear.py:446-493).
 */
int sla2h_lin_fwd3(const void* qphi, const void* comp, const void* o_s, const float* alpha,
                   int alpha_stride, int dtype, int B, int H, int64_t L, int D, int bq,
                   float eps_l, void* o, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SLA2H_H */
