"""CPU restatement of the SLA2 INT8 cube-attention hot path (test infrastructure only).

Bit-exact parts (quantisation, pooling, router scores, top-k) are numpy fp32
with every sum in a fixed sequential order and no fused multiply-add: numpy
rounds each elementwise fp32 operation separately, exactly as the gfx950
kernels compiled with -ffp-contract=off do.  Floating-point parts (phi,
states, attention, linear branch) are torch CPU fp32 following the reference
kernels operation by operation, including the 16-bit rounding of the MMA
operands P and t.  Dense fp64 forms at the bottom serve only to pin the
blockwise restatement on tiny inputs.

All inputs are CPU tensors / arrays holding the fp32 values of the 16-bit
data (bf16 or fp16), tile-major token order, shape (B, H, L, D).
"""

import math

import numpy as np
import torch
import torch.nn.functional as F

E = 64
LOG2E = 1.4426950408889634
EPS_L = 1e-5
_F32 = np.float32


def _np(x):
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().float().numpy()
    return np.asarray(x, dtype=np.float32)


def _pad_rows(x, rows):
    pad = rows - x.shape[-2]
    if pad == 0:
        return x
    z = np.zeros(x.shape[:-2] + (pad, x.shape[-1]), dtype=x.dtype)
    return np.concatenate([x, z], axis=-2)


# ---------------------------------------------------------------------------
# INT8 block quantisation -- models/sla2_vendor/kernel_sparse_qat.py:128-141
#   s = max|x| / 127 + 1e-12 (fp32 ops), q = round_half_away(x / s)
# ---------------------------------------------------------------------------
def round_half_away(y):
    """Round to nearest, ties away from zero (libdevice.round), exact in fp32."""
    a = np.abs(y)
    f = np.floor(a)
    r = f + ((a - f) >= _F32(0.5)).astype(np.float32)
    return np.where(y < 0, -r, r)


def quantize_blocks(x, block=E):
    """x (..., L, D) -> (q int8 (..., L, D), s fp32 (..., ceil(L/block)))."""
    x = _np(x)
    L, D = x.shape[-2:]
    nb = -(-L // block)
    xb = _pad_rows(x, nb * block).reshape(x.shape[:-2] + (nb, block, D))
    amax = np.abs(xb).max(axis=(-2, -1))
    s = (amax / _F32(127.0)).astype(np.float32) + _F32(1e-12)
    y = xb / s[..., None, None]
    q = round_half_away(y).astype(np.int8)
    return q.reshape(x.shape[:-2] + (nb * block, D))[..., :L, :], s.astype(np.float32)


# ---------------------------------------------------------------------------
# Router -- models/mla_video_sparse_jvp.py:506-566 (route_tiles_fast) with the
# canonical fp32 order: per-channel sequential sum over rows, / count;
# projections and scores as sequential fp32 dots (mul, then add).
# ---------------------------------------------------------------------------
def pool_tiles(x, nblocks, count_len, block=E):
    """Mean of each of the first `nblocks` blocks over its rows < count_len."""
    x = _np(x)
    D = x.shape[-1]
    out = np.zeros(x.shape[:-2] + (nblocks, D), dtype=np.float32)
    for b in range(nblocks):
        cnt = min(block, count_len - b * block)
        acc = np.zeros(x.shape[:-2] + (D,), dtype=np.float32)
        for r in range(cnt):
            acc = acc + x[..., b * block + r, :]
        out[..., b, :] = acc / _F32(cnt)
    return out


def project_pool(p, proj):
    """p (..., n, D) @ proj^T with a sequential fp32 dot: out[e] = sum_d p[d] proj[e, d]."""
    if proj is None:
        return p
    proj = _np(proj)
    acc = np.zeros(p.shape[:-1] + (proj.shape[0],), dtype=np.float32)
    for d in range(p.shape[-1]):
        acc = acc + p[..., d:d + 1] * proj[:, d]
    return acc


def route_scores(qp, kp, scale):
    """pc[..., m, n] = (sum_d qp[m, d] kp[n, d]) * scale, sequential fp32."""
    acc = np.zeros(qp.shape[:-1] + (kp.shape[-2],), dtype=np.float32)
    for d in range(qp.shape[-1]):
        acc = acc + qp[..., :, d:d + 1] * kp[..., None, :, d]
    return acc * _F32(scale)


def score_keys(pc):
    """Total order of torch.topk on fp32 (NaN largest, -0 == +0), ties to lower index."""
    u = np.ascontiguousarray(pc, dtype=np.float32).view(np.uint32).copy()
    u[np.isnan(pc)] = 0x7FC00000
    u[u == 0x80000000] = 0
    ordk = np.where(u & 0x80000000, ~u, u | 0x80000000).astype(np.uint64)
    idx = np.arange(pc.shape[-1], dtype=np.uint64)
    return (ordk << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)


def topk_rows(pc, T):
    """Indices of the T largest per row, in descending score order (int32)."""
    keys = score_keys(pc)
    order = np.argsort(keys, axis=-1, kind="stable")[..., ::-1]
    return np.ascontiguousarray(order[..., :T]).astype(np.int32)


def topk_count(topk_frac, Np):
    return max(1, min(Np, int(topk_frac * Np)))


def route(q, k, topk_frac, Np, prefix_len=0, proj_q=None, proj_k=None, T=None):
    """Returns (lut int32 (B,H,Mb,T), T, qpool (B,H,Mb,D), kpool (B,H,Np,D))."""
    q, k = _np(q), _np(k)
    L, D = q.shape[-2:]
    Mb = -(-L // E)
    qp = project_pool(pool_tiles(q, Mb, L), proj_q)
    kp = project_pool(pool_tiles(k, Np, Np * E), proj_k)
    pc = route_scores(qp, kp, D ** -0.5)
    T = topk_count(topk_frac, Np) if T is None else T
    return topk_rows(pc, T), T, qp, kp


# ---------------------------------------------------------------------------
# Tile permutation -- models/mla_video_sparse_jvp.py:61-91
# ---------------------------------------------------------------------------
def tile_permutation(grid, tile, prefix_len):
    Tg, Hh, Ww = grid
    tt, th, tw = tile
    assert Tg % tt == 0 and Hh % th == 0 and Ww % tw == 0
    idx = np.arange(Tg * Hh * Ww).reshape(Tg // tt, tt, Hh // th, th, Ww // tw, tw)
    idx = idx.transpose(0, 2, 4, 1, 3, 5).reshape(-1) + prefix_len
    perm = np.concatenate([idx, np.arange(prefix_len)])
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.size)
    return perm, inv, (Tg // tt) * (Hh // th) * (Ww // tw)


# ---------------------------------------------------------------------------
# phi-states -- models/sla2_cube_qat.py:911-958 and the sums at :645-648
# ---------------------------------------------------------------------------
def phi_jvp(x, dx=None):
    """phi = softmax over D (fp32), dphi = phi * (dx - <phi, dx>)."""
    x = x.float()
    mx = x.amax(-1, keepdim=True)
    ex = torch.exp(x - mx)
    phi = ex / ex.sum(-1, keepdim=True)
    if dx is None:
        return phi, None
    dx = dx.float()
    return phi, phi * (dx - (phi * dx).sum(-1, keepdim=True))


def phi_states(k, v, Np, dk=None, dv=None):
    """Per-video-tile states and their sums over the Np tiles (fp32)."""
    B, H, L, D = k.shape
    kv = k[:, :, :Np * E].float().reshape(B, H, Np, E, D)
    vv = v[:, :, :Np * E].float().reshape(B, H, Np, E, D)
    phi, dphi = phi_jvp(kv, None if dk is None else dk[:, :, :Np * E].reshape(B, H, Np, E, D))
    st = {"Hb": torch.einsum("bhnrd,bhnrv->bhndv", phi, vv), "zb": phi.sum(3)}
    if dk is not None:
        dvv = dv[:, :, :Np * E].float().reshape(B, H, Np, E, D)
        st["dHb"] = (torch.einsum("bhnrd,bhnrv->bhndv", dphi, vv)
                     + torch.einsum("bhnrd,bhnrv->bhndv", phi, dvv))
        st["dzb"] = dphi.sum(3)
    st["Hall"] = st["Hb"].sum(2)
    st["zall"] = st["zb"].sum(2)
    if dk is not None:
        st["dHall"] = st["dHb"].sum(2)
        st["dzall"] = st["dzb"].sum(2)
    return st


# ---------------------------------------------------------------------------
# The fused op -- models/sla2_cube_qat.py:448-602 (_cube_fused_jvp_kernel)
# ---------------------------------------------------------------------------
def _tiles(x, nb):
    B, H, L, D = x.shape
    pad = nb * E - L
    if pad:
        x = torch.cat([x, x.new_zeros(B, H, pad, D)], 2)
    return x.reshape(B, H, nb, E, D)


def _gather_tiles(xt, idx):
    """xt (B,H,nb,E,D), idx (B,H,Mb) -> (B,H,Mb,E,D)."""
    B, H, Mb = idx.shape
    ix = idx.long().view(B, H, Mb, 1, 1).expand(B, H, Mb, xt.shape[3], xt.shape[4])
    return torch.gather(xt, 2, ix)


def cube_jvp(q, k, v, dq, dk, dv, alpha, lut, Np, prefix_len, quant=None, states=None,
             t16=torch.bfloat16, sparse_only=False):
    """Blockwise restatement of the fused INT8 op and its JVP.

    q..dv: (B,H,L,D) float tensors holding the 16-bit values (dq,dk,dv None =
    primal only).  alpha (H, Mb) after the sigmoid.  lut (B,H,Mb,T) ids.
    quant: optional (q8, qs, k8, ks) (numpy or torch); computed when None.
    t16: the 16-bit type of the MMA operands p and t.
    Returns (o, do) fp32 (B,H,L,D); do is None for primal only.
    """
    B, H, L, D = q.shape
    nb = -(-L // E)
    Mb = nb
    n_tail = nb - Np
    tan = dq is not None
    lut = torch.as_tensor(np.asarray(lut)).long()
    T = lut.shape[-1]
    if quant is None:
        q8, qs = quantize_blocks(q)
        k8, ks = quantize_blocks(k)
    else:
        q8, qs, k8, ks = quant
    q8, k8 = (torch.as_tensor(np.asarray(t)).double() for t in (q8, k8))
    qs, ks = (torch.as_tensor(np.asarray(t)).float() for t in (qs, ks))
    scale = float(np.float32(D ** -0.5))
    c_log2 = float(np.float32(scale) * np.float32(LOG2E))
    qf, kf, vf = q.float(), k.float(), v.float()

    Qt = _tiles(qf, nb)
    Q8t = _tiles(q8, nb)
    K8t, Kt, Vt = _tiles(k8, nb), _tiles(kf, nb), _tiles(vf, nb)
    if tan:
        dQt, dKt, dVt = _tiles(dq.float(), nb), _tiles(dk.float(), nb), _tiles(dv.float(), nb)

    m_i = torch.full((B, H, Mb, E), -math.inf)
    l_i = torch.zeros(B, H, Mb, E)
    mu = torch.zeros(B, H, Mb, E)
    acc_o = torch.zeros(B, H, Mb, E, D)
    acc_do = torch.zeros(B, H, Mb, E, D) if tan else None
    lin = not sparse_only
    if lin:
        if states is None:
            states = phi_states(k, v, Np, dk, dv)
        hc = states["Hall"][:, :, None].expand(B, H, Mb, D, D).clone().float()
        zc = states["zall"][:, :, None].expand(B, H, Mb, D).clone().float()
        if tan:
            dhc = states["dHall"][:, :, None].expand(B, H, Mb, D, D).clone().float()
            dzc = states["dzall"][:, :, None].expand(B, H, Mb, D).clone().float()

    qsb = qs[:, :, :Mb]
    key_pos = torch.arange(E)
    for j in range(T + n_tail):
        if j < T:
            n = lut[..., j]
        else:
            n = torch.full((B, H, Mb), Np + (j - T), dtype=torch.long)
        k8n = _gather_tiles(K8t, n)
        s_int = torch.matmul(Q8t, k8n.transpose(-1, -2))       # exact in fp64
        sk = torch.gather(ks, 2, n)                               # (B,H,Mb)
        sqk = (qsb * sk)[..., None, None]
        s2 = (s_int.float() * sqk) * c_log2
        valid = (n[..., None] * E + key_pos) < L                 # (B,H,Mb,E)
        s2 = s2.masked_fill(~valid[..., None, :], -math.inf)
        m_new = torch.maximum(m_i, s2.amax(-1))
        al = torch.exp2(m_i - m_new)
        p = torch.exp2(s2 - m_new[..., None])
        l_i = l_i * al + p.sum(-1)
        vn = _gather_tiles(Vt, n)
        pc = p.to(t16).float()
        acc_o = acc_o * al[..., None] + torch.matmul(pc, vn)
        if tan:
            kn, dkn, dvn = _gather_tiles(Kt, n), _gather_tiles(dKt, n), _gather_tiles(dVt, n)
            ds = (torch.matmul(dQt, kn.transpose(-1, -2))
                  + torch.matmul(Qt, dkn.transpose(-1, -2))) * scale
            t = p * ds
            mu = mu * al + t.sum(-1)
            tcl = t.clamp(-60000.0, 60000.0) if t16 == torch.float16 else t
            tc = tcl.to(t16).float()
            acc_do = acc_do * al[..., None] + torch.matmul(tc, vn) + torch.matmul(pc, dvn)
        m_i = m_new
        if lin and j < T:
            ix4 = n.view(B, H, Mb, 1, 1).expand(B, H, Mb, D, D)
            ix3 = n.view(B, H, Mb, 1).expand(B, H, Mb, D)
            hc = hc - torch.gather(states["Hb"].float(), 2, ix4)
            zc = zc - torch.gather(states["zb"].float(), 2, ix3)
            if tan:
                dhc = dhc - torch.gather(states["dHb"].float(), 2, ix4)
                dzc = dzc - torch.gather(states["dzb"].float(), 2, ix3)

    o = acc_o / l_i[..., None]
    do = (acc_do / l_i[..., None] - (mu / l_i)[..., None] * o) if tan else None
    if lin:
        qphi, dqphi = phi_jvp(Qt, dQt if tan else None)
        num = torch.matmul(qphi, hc)
        den = (qphi * zc[..., None, :]).sum(-1)
        den = torch.where(den >= 0, den + EPS_L, den - EPS_L)
        o_l = num / den[..., None]
        a = torch.as_tensor(alpha).float().reshape(1, H, Mb, 1, 1)
        if tan:
            dnum = torch.matmul(dqphi, hc) + torch.matmul(qphi, dhc)
            dden = (dqphi * zc[..., None, :]).sum(-1) + (qphi * dzc[..., None, :]).sum(-1)
            do_l = (dnum - o_l * dden[..., None]) / den[..., None]
            do = a * do + (1.0 - a) * do_l
        o = a * o + (1.0 - a) * o_l
    o = o.reshape(B, H, Mb * E, D)[:, :, :L]
    if do is not None:
        do = do.reshape(B, H, Mb * E, D)[:, :, :L]
    return o, do


# ---------------------------------------------------------------------------
# Dense fp64 forms (tiny L only) used to pin the blockwise restatement.
# ---------------------------------------------------------------------------
def block_mask(lut, Np, L, prefix_len):
    """(B,H,L,L) {0,1} sparse mask (routed tiles + prefix columns) and complement."""
    lut = torch.as_tensor(np.asarray(lut)).long()
    B, H, Mb, T = lut.shape
    mc = torch.zeros(B, H, Mb, Np, dtype=torch.float64)
    mc.scatter_(-1, lut, 1.0)
    m = mc.repeat_interleave(E, dim=-2)[:, :, :L].repeat_interleave(E, dim=-1)
    m = torch.cat([m, torch.ones(B, H, L, L - Np * E, dtype=torch.float64)], -1)
    comp = 1.0 - m
    comp[..., Np * E:] = 0.0
    return m, comp


def dense_op(S, v, q, k, alpha, m, comp, Np, eps=EPS_L):
    """o = a softmax_m(S) v + (1 - a) [phi(q) phi(k)^T * comp] v / (sum + eps), fp64.

    S is the (already scaled) score matrix.  Mirrors mvs_dense_ref
    (models/mla_video_sparse_jvp.py:457-498) with S passed in, so that the
    INT8 primal scores and the straight-through tangent can be fed to
    torch.func.jvp.
    """
    B, H, L, D = v.shape
    p = torch.softmax(S.masked_fill(m <= 0, -math.inf), dim=-1)
    o_s = p @ v
    w = (torch.softmax(q, -1) @ torch.softmax(k, -1).transpose(-1, -2)) * comp
    o_l = (w @ v) / (w.sum(-1, keepdim=True) + eps)
    Mb = -(-L // E)
    reps = torch.tensor([E] * (Mb - 1) + [L - (Mb - 1) * E])
    a = torch.as_tensor(alpha, dtype=torch.float64).repeat_interleave(reps, -1).view(1, H, L, 1)
    return a * o_s + (1.0 - a) * o_l


def dense_jvp(q, k, v, dq, dk, dv, alpha, lut, Np, prefix_len, quant=None):
    """fp64 (o, do): primal scores from the dequantised INT8 Q/K, tangent scores
    (dq k^T + q dk^T) * scale from the unquantised values (straight-through),
    differentiated by torch.func.jvp through dense_op."""
    B, H, L, D = q.shape
    if quant is None:
        q8, qs = quantize_blocks(q)
        k8, ks = quantize_blocks(k)
    else:
        q8, qs, k8, ks = quant
    deq = lambda x8, s: (torch.as_tensor(np.asarray(x8)).double()
                         * torch.as_tensor(np.asarray(s)).double().repeat_interleave(E, -1)[..., :L, None])
    qd, kd = deq(q8, qs), deq(k8, ks)
    scale = D ** -0.5
    qq, kk, vv = q.double(), k.double(), v.double()
    S = (qd @ kd.transpose(-1, -2)) * scale
    m, comp = block_mask(lut, Np, L, prefix_len)
    if dq is None:
        return dense_op(S, vv, qq, kk, alpha, m, comp, Np), None
    dS = (dq.double() @ kk.transpose(-1, -2) + qq @ dk.double().transpose(-1, -2)) * scale
    f = lambda S_, v_, q_, k_: dense_op(S_, v_, q_, k_, alpha, m, comp, Np)
    return torch.func.jvp(f, (S, vv, qq, kk), (dS, dv.double(), dq.double(), dk.double()))


# ---------------------------------------------------------------------------
# Training-forward semantics (b): _CubeQATFunction.forward
# (models/sla2_cube_qat.py:696-751) = _attn_fwd_qat (kernel_sparse_qat.py:28-117)
# + kphi / _precompute_global (kernel_linear.py:305-313) + _lin_fwd2 in its
# state or score form (kernel_linear.py:205-302) + the alpha mix in 16-bit.
# ---------------------------------------------------------------------------
def quantize_blocks_trunc(x, block=E):
    """In-kernel quantisation of _attn_fwd_qat (kernel_sparse_qat.py:56-58, 88-90,
    106-107): s = max|x|/127 + 1e-12, q = int(fl32(fl32(x / s) + 0.5*sign(x)))
    truncated toward zero (sign(+-0) = +1).  x (..., L, D) -> (q int8, s fp32)."""
    x = _np(x)
    L, D = x.shape[-2:]
    nb = -(-L // block)
    xb = _pad_rows(x, nb * block).reshape(x.shape[:-2] + (nb, block, D))
    amax = np.abs(xb).max(axis=(-2, -1))
    s = (amax / _F32(127.0)).astype(np.float32) + _F32(1e-12)
    y = (xb / s[..., None, None]).astype(np.float32)
    y = (y + np.where(xb >= 0, _F32(0.5), _F32(-0.5))).astype(np.float32)
    q = np.trunc(y).astype(np.int8)
    return q.reshape(x.shape[:-2] + (nb * block, D))[..., :L, :], s.astype(np.float32)


def _round16(x, t16):
    return x.to(t16).float()


def _expand_1d(lut, alpha, bq, nb):
    """Query blocks of bq rows -> 64-row sub-blocks sharing their block's LUT row and alpha."""
    r = bq // E
    lut = torch.as_tensor(np.asarray(lut)).repeat_interleave(r, dim=2)[:, :, :nb]
    alpha = torch.as_tensor(alpha).repeat_interleave(r, dim=-1)[:, :nb]
    return lut, alpha


def train_fwd(q, k, v, alpha, lut, Np, prefix_len, t16=torch.bfloat16, eps=EPS_L, int8=True,
              bq=E, score_form=None):
    """Training-forward semantics (b), blockwise, CPU.

    q, k, v: (B,H,L,D) float tensors holding 16-bit values.  alpha: (H, Mb)
    after the sigmoid.  lut: (B,H,Mb,T) routed video tiles; the n_tail prefix
    blocks are appended (lut_aug).  Returns dict with o (16-bit values, the
    module output), o_s, o_l (16-bit values), lse (fp32, log2 domain), qphi,
    den (the signed-epsilon denominator), htot (16-bit values), ztot.
    bq > 64: the 1-D SLA2 module's forward (_sparse_attention_qat,
    models/sla2_vendor/kernel_sparse_qat.py:265-293, and
    _complement_linear_attention, models/sla2_vendor/kernel_linear.py:340-366):
    query blocks of bq rows (LUT rows, alpha and, with int8, the Q scale per
    block), Np = Nb key blocks and no prefix tail; int8=False: 16-bit scores
    and O += round16(P).V.
    score_form: the linear branch's form; None selects it as the reference's
    callers do (score form while the augmented LUT has at most 4 columns,
    models/sla2_cube_qat.py:424, 739; models/sla2_vendor/kernel_linear.py:357),
    True / False force the score / state form.
    """
    B, H, L, D = q.shape
    nb = -(-L // E)
    Mb = nb
    if bq != E:
        lut, alpha = _expand_1d(lut, alpha, bq, nb)
    n_tail = nb - Np
    lut = torch.as_tensor(np.asarray(lut)).long()
    tails = torch.arange(Np, Np + n_tail).view(1, 1, 1, -1).expand(B, H, Mb, n_tail)
    lut_aug = torch.cat([lut, tails], -1)
    J = lut_aug.shape[-1]
    if not int8:   # 16-bit operands: the "int8" tensors below hold the 16-bit values, scales 1
        q8, k8, v8 = (torch.as_tensor(x).float().numpy() for x in (q, k, v))
        qs = ks = vs = np.ones((B, H, nb), dtype=np.float32)
    else:   # Q per bq rows (the kernel's BLOCK_M), K and V per 64-row block
        q8, qs = quantize_blocks_trunc(q, bq)
        if bq != E:
            qs = np.repeat(qs, bq // E, axis=-1)[..., :nb]
        k8, ks = quantize_blocks_trunc(k)
        v8, vs = quantize_blocks_trunc(v)
    q8t = _tiles(torch.as_tensor(q8).double(), nb)
    k8t = _tiles(torch.as_tensor(k8).double(), nb)
    v8t = _tiles(torch.as_tensor(v8).double(), nb)
    qs, ks, vs = (torch.as_tensor(t).float() for t in (qs, ks, vs))
    scale = float(np.float32(D ** -0.5))
    c2 = float(np.float32(scale * LOG2E))
    rows = torch.arange(nb * E).view(nb, E)
    m_i = torch.full((B, H, Mb, E), -math.inf)
    l_i = torch.zeros(B, H, Mb, E)
    o_s = torch.zeros(B, H, Mb, E, D)
    for j in range(J):
        n = lut_aug[..., j]                                   # (B,H,Mb)
        kt = _gather_tiles(k8t, n)                            # (B,H,Mb,E,D)
        vt = _gather_tiles(v8t, n)
        skn = torch.gather(ks, 2, n)                          # (B,H,Mb)
        svn = torch.gather(vs, 2, n)
        si = torch.matmul(q8t[:, :, :Mb], kt.transpose(-1, -2)).float()  # exact ints
        qk = si * (qs[:, :, :Mb] * skn)[..., None, None]
        qk = qk * c2
        valid = (rows[n] < L)                                 # (B,H,Mb,E) key rows
        qk = qk.masked_fill(~valid[..., None, :], -math.inf)
        local_m = qk.amax(-1)
        new_m = torch.maximum(m_i, local_m)
        p = torch.exp2(qk - new_m[..., None])
        l_ij = p.sum(-1)
        al = torch.exp2(m_i - new_m)
        o_s = o_s * al[..., None]
        if int8:
            p8 = torch.trunc(p * 127.0 + 0.5)
            pv = torch.matmul(p8.double(), vt).float()
            o_s = o_s + pv * (svn / 127.0)[..., None, None]
        else:
            o_s = o_s + torch.matmul(_round16(p, t16).double(), vt).float()
        l_i = l_i * al + l_ij
        m_i = new_m
    o_s = o_s / l_i[..., None]
    lse = m_i + torch.log2(l_i)
    o_s = o_s.reshape(B, H, Mb * E, D)[:, :, :L]
    lse = lse.reshape(B, H, Mb * E)[:, :, :L]
    o_s16 = _round16(o_s, t16)
    qphi = _round16(torch.softmax(q.float(), -1), t16)
    kphi = _round16(torch.softmax(k.float(), -1), t16)
    vf = v.float()
    htot = _round16(kphi.transpose(-1, -2) @ vf, t16)          # (B,H,D,D)
    ztot = kphi.sum(-2)                                        # (B,H,D)
    kpt, vvt = _tiles(kphi, nb), _tiles(vf, nb)
    qpt = _tiles(qphi, nb)
    if score_form is None:
        score_form = J <= 4
    if score_form:
        # _lin_fwd2 with SCORE_FORM (kernel_linear.py:260-272): the selected
        # tiles are subtracted in the score domain, w = phi(Q) phi(K_j)^T in
        # fp32, rounded to 16 bits for the product with V_j, unrounded in den
        qp = qpt[:, :, :Mb]                                    # (B,H,Mb,E,D)
        num = qp @ htot[:, :, None]
        den = (qp * ztot[:, :, None, None, :]).sum(-1)
        for j in range(J):
            n = lut_aug[..., j]
            kp, vv = _gather_tiles(kpt, n), _gather_tiles(vvt, n)
            w = qp @ kp.transpose(-1, -2)                      # (B,H,Mb,E,E)
            num = num - _round16(w, t16) @ vv
            den = den - w.sum(-1)
    else:
        # state form (kernel_linear.py:274-285)
        hi = htot[:, :, None].expand(B, H, Mb, D, D).clone()
        zi = ztot[:, :, None].expand(B, H, Mb, D).clone()
        for j in range(J):
            n = lut_aug[..., j]
            kp, vv = _gather_tiles(kpt, n), _gather_tiles(vvt, n)
            hi = hi - kp.transpose(-1, -2) @ vv
            zi = zi - kp.sum(-2)
        num = qpt[:, :, :Mb] @ _round16(hi, t16)              # (B,H,Mb,E,D)
        den = (qpt[:, :, :Mb] * zi[..., None, :]).sum(-1)
    den = torch.where(den >= 0, den + eps, den - eps)
    o_l = (num / den[..., None]).reshape(B, H, Mb * E, D)[:, :, :L]
    den = den.reshape(B, H, Mb * E)[:, :, :L]
    o_l16 = _round16(o_l, t16)
    a = _round16(alpha.float()[None, :, :, None, None].expand(B, H, Mb, E, 1)
                 .reshape(B, H, Mb * E, 1)[:, :, :L], t16)
    o = _round16(_round16(a * o_s16, t16) + _round16(_round16(1.0 - a, t16) * o_l16, t16), t16)
    return {"o": o, "o_s": o_s16, "o_l": o_l16, "lse": lse, "qphi": qphi, "den": den,
            "htot": htot, "ztot": ztot}


def train_bwd(q, k, v, alpha, lut, Np, prefix_len, fwd, do, t16=torch.bfloat16, bq=E,
              variant="cube"):
    """Training backward (straight-through estimator), blockwise, CPU.

    Restates _CubeQATFunction.backward (models/sla2_cube_qat.py:753-832) and its
    kernels: _bwd_split_kernel (:838-872), _attn_bwd_preprocess / _attn_bwd_dq
    (models/sla2_vendor/sla_kernel.py:89-184), _sparse_bwd_dkdv_lut
    (models/sla2_cube_qat.py:986-1042), _lin_bwd_dq
    (models/sla2_vendor/kernel_linear.py:85-138), _lin_bwd_dkdv_lut
    (models/sla2_cube_qat.py:1045-1104), _phi_chain_add_kernel (:875-904).

    The sparse branch is re-differentiated with the UNQUANTISED q, k, v in
    16-bit, p = exp2(min(q.k * scale*log2e - lse, 4)) with the INT8 forward's
    lse, delta = rowsum(o_s * do_s); 16-bit rounding of ds, p (for dv), the
    stored dq_s/dk_s/dv_s; saturation at +-60000 where the reference clamps.
    fwd: the train_fwd dict (o_s, o_l, lse, den, qphi, htot, ztot); do (B,H,L,D)
    the output gradient; alpha (H, Mb) after the sigmoid.
    t16=None: exact mode (float64, no rounding, no clamps), in which the result
    is the exact gradient of the op whose forward quantities fwd holds.
    Returns dict dq, dk, dv (B,H,L,D), d_alpha (H, Mb; the gradient with respect
    to the alpha LOGITS) and the intermediates dq_s, dk_s, dv_s, dqphi, dkphi,
    dv_l, delta.  LUT rows are assumed free of duplicates (top-k rows are).

    bq > 64: query blocks of bq rows (LUT rows and alpha per block).
    variant="1d": the rounding points of the 1-D SLA2 module's backward, where
    the mix and the phi maps are torch autograd ops on fp16 tensors
    (models/sla2_vendor/core.py:168-176) and the linear branch is
    _complement_linear_attention.backward (kernel_linear.py:368-393):
    do_s = r16(do a16), do_l = r16(do r16(1 - a16)) with a16 = r16(a); dqphi and
    dkphi stored in 16 bits; _lin_bwd_dkdv without saturation; the softmax
    backward rounded to 16 bits and added to the 16-bit sparse gradient.
    """
    one_d = variant == "1d"
    B_, H_, L_, D_ = q.shape
    if bq != E:
        nb_ = -(-L_ // E)
        mq = -(-L_ // bq)
        alpha_q = torch.as_tensor(alpha)
        lut, alpha = _expand_1d(lut, alpha, bq, nb_)
    exact = t16 is None
    dt = torch.float64 if exact else torch.float32
    r16 = (lambda x: x) if exact else (lambda x: x.to(t16).to(dt))
    sat = (lambda x: x) if exact else (lambda x: x.clamp(-60000.0, 60000.0))
    B, H, L, D = q.shape
    nb = -(-L // E)
    Mb = nb
    n_tail = nb - Np
    lut = torch.as_tensor(np.asarray(lut)).long()
    tails = torch.arange(Np, Np + n_tail).view(1, 1, 1, -1).expand(B, H, Mb, n_tail)
    lut_aug = torch.cat([lut, tails], -1)
    J = lut_aug.shape[-1]
    cv = lambda x: torch.as_tensor(x).to(dt)
    q, k, v, do = cv(q), cv(k), cv(v), cv(do)
    o_s, o_l, lse, den, qphi = (cv(fwd[n]) for n in ("o_s", "o_l", "lse", "den", "qphi"))
    htot, ztot = cv(fwd["htot"]), cv(fwd["ztot"])
    a_blk = cv(alpha)                                          # (H, Mb)
    rows = torch.arange(nb * E)
    a_rows = a_blk[:, (rows[:L] // E)].view(1, H, L, 1)
    if one_d:
        a16 = r16(a_rows)
        do_s, do_l = r16(do * a16), r16(do * r16(1.0 - a16))
    else:
        do_s, do_l = r16(do * a_rows), r16(do * (1.0 - a_rows))
    segr = (do * (o_s - o_l)).sum(-1)                          # (B,H,L)
    seg = _tiles(segr[..., None], nb).sum((-2, -1)).sum(0)     # (H, Mb)
    if bq != E:   # per query block of bq rows
        seg = torch.stack([seg[:, i * (bq // E):(i + 1) * (bq // E)].sum(-1) for i in range(mq)], -1)
        a_blk = cv(alpha_q)
    d_alpha = seg * a_blk * (1.0 - a_blk)
    delta = (o_s * do_s).sum(-1)
    scale = D ** -0.5
    c = scale * LOG2E if exact else float(np.float32(scale * LOG2E))
    qt, kt, vt, dost = (_tiles(x, nb) for x in (q, k, v, do_s))
    pad1 = lambda x, val: torch.cat([x, x.new_full((B, H, nb * E - L), val)], -1).view(B, H, nb, E)
    lse_t, delta_t = pad1(lse, math.inf), pad1(delta, 0.0)
    key_rows = rows.view(nb, E)
    dq_acc = torch.zeros(B, H, Mb, E, D, dtype=dt)
    dk_acc = torch.zeros(B, H, nb, E, D, dtype=dt)
    dv_acc = torch.zeros(B, H, nb, E, D, dtype=dt)
    ix = lambda n: n.view(B, H, Mb, 1, 1).expand(B, H, Mb, E, D)
    for j in range(J):
        n = lut_aug[..., j]
        kn, vn = _gather_tiles(kt, n), _gather_tiles(vt, n)
        x = (qt @ kn.transpose(-1, -2)) * c - lse_t[..., None]
        p = torch.exp2(x if exact else torch.clamp(x, max=4.0))
        p = p.masked_fill(~(key_rows[n] < L)[..., None, :], 0.0)
        dp = dost @ vn.transpose(-1, -2)
        ds16 = r16(sat(p * (dp - delta_t[..., None])))
        dq_acc += ds16 @ kn
        dk_acc.scatter_add_(2, ix(n), ds16.transpose(-1, -2) @ qt)
        dv_acc.scatter_add_(2, ix(n), r16(p).transpose(-1, -2) @ dost)
    untile = lambda x: x.reshape(B, H, nb * E, -1)[:, :, :L]
    dq_s = r16(untile(dq_acc) * scale)
    dk_s = r16(untile(dk_acc) * scale)
    dv_s = r16(untile(dv_acc))

    # linear branch
    g = do_l / den[..., None]
    s = (do_l * o_l).sum(-1) / den
    dhtot = qphi.transpose(-1, -2) @ g                         # (B,H,D,D)
    dztot = -(qphi * s[..., None]).sum(-2)                     # (B,H,D)
    kphi = torch.softmax(k, -1) if exact else r16(torch.softmax(k.float(), -1).to(dt))
    kpt, vvt = _tiles(kphi, nb), _tiles(v, nb)
    hi = htot[:, :, None].expand(B, H, Mb, D, D).clone()
    zi = ztot[:, :, None].expand(B, H, Mb, D).clone()
    for j in range(J):
        n = lut_aug[..., j]
        kp, vv = _gather_tiles(kpt, n), _gather_tiles(vvt, n)
        hi -= kp.transpose(-1, -2) @ vv
        zi -= kp.sum(-2)
    g16 = r16(sat(g))
    g16t, st, qpt = _tiles(g16, nb), pad1(s, 0.0), _tiles(qphi, nb)
    dqphi = g16t @ r16(hi).transpose(-1, -2) - st[..., None] * zi[..., None, :]
    dqphi = untile(dqphi)
    if one_d:
        dqphi = r16(dqphi)
        g16t = _tiles(r16(g), nb)
    pm = qpt.transpose(-1, -2) @ g16t                          # (B,H,Mb,D,D)
    pz = (qpt * st[..., None]).sum(-2)                         # (B,H,Mb,D)
    dh = dhtot[:, :, None].expand(B, H, nb, D, D).clone()
    dz = dztot[:, :, None].expand(B, H, nb, D).clone()
    for j in range(J):
        n = lut_aug[..., j]
        dh.scatter_add_(2, ix(n)[..., :D, :], -pm)
        dz.scatter_add_(2, n.view(B, H, Mb, 1).expand(B, H, Mb, D), pz)
    dh16 = r16(dh) if one_d else r16(sat(dh))
    dkphi = untile(vvt @ dh16.transpose(-1, -2) + dz[..., None, :])
    dv_l = untile(kpt @ dh16)

    chain = lambda phi, dphi: phi * (dphi - (phi * dphi).sum(-1, keepdim=True))
    if one_d:
        dkphi, dv_l = r16(dkphi), r16(dv_l)
        dq = r16(dq_s + r16(chain(qphi, dqphi)))
        dk = r16(dk_s + r16(chain(kphi, dkphi)))
        dv = r16(dv_s + dv_l)
    else:
        dq = r16(sat(dq_s + chain(qphi, dqphi)))
        dk = r16(sat(dk_s + chain(kphi, dkphi)))
        dv = r16(sat(dv_s + dv_l))
    return {"dq": dq, "dk": dk, "dv": dv, "d_alpha": d_alpha, "dq_s": dq_s, "dk_s": dk_s,
            "dv_s": dv_s, "dqphi": dqphi, "dkphi": dkphi, "dv_l": dv_l, "delta": delta}


def train_dense_f64(q, k, v, alpha_logit, lut, Np, prefix_len, eps=EPS_L, bq=E):
    """Differentiable float64 restatement of the training op WITHOUT quantisation
    (the straight-through view): masked softmax over the augmented-LUT tiles,
    complement linear attention over the other video tiles, sigmoid mix.

    Returns (o, fwd) where fwd holds the forward quantities train_bwd consumes
    (o_s, o_l, lse in log2, den, qphi, htot, ztot), detached.  Dense O(L^2):
    tiny inputs only.
    """
    B, H, L, D = q.shape
    nb = -(-L // E)
    n_tail = nb - Np
    lut = torch.as_tensor(np.asarray(lut)).long()
    mq = lut.shape[2]
    tails = torch.arange(Np, Np + n_tail).view(1, 1, 1, -1).expand(B, H, mq, n_tail)
    lut_aug = torch.cat([lut, tails], -1)
    sel = torch.zeros(B, H, mq, nb, dtype=torch.bool)
    sel.scatter_(3, lut_aug, True)
    blk = torch.arange(L) // E
    qblk = torch.arange(L) // bq
    allowed = sel[:, :, qblk][:, :, :, blk]                    # (B,H,L,L)
    s = (q @ k.transpose(-1, -2)) * D ** -0.5
    s = s.masked_fill(~allowed, -math.inf)
    o_s = torch.softmax(s, -1) @ v
    lse = torch.logsumexp(s, -1) * LOG2E
    qphi, kphi = torch.softmax(q, -1), torch.softmax(k, -1)
    w = (qphi @ kphi.transpose(-1, -2)) * (~allowed)
    den0 = w.sum(-1)
    den = torch.where(den0 >= 0, den0 + eps, den0 - eps)
    o_l = (w @ v) / den[..., None]
    a = torch.sigmoid(alpha_logit)[:, qblk].view(1, H, L, 1)
    o = a * o_s + (1 - a) * o_l
    fwd = {"o_s": o_s, "o_l": o_l, "lse": lse, "den": den, "qphi": qphi,
           "htot": kphi.transpose(-1, -2) @ v, "ztot": kphi.sum(-2)}
    return o, {n: t.detach() for n, t in fwd.items()}


# ---------------------------------------------------------------------------
# 1-D SLA2 blocks (query blocks of bq rows, key blocks of bk = 64 rows):
# route_blocks and sla2_mla_jvp (models/sla2_mla_jvp.py:51-99, 108-385).
# ---------------------------------------------------------------------------
def infer_1d(q, k, v, alpha, lut, bq, int8=True, qblock=None, t16=torch.float16, eps=EPS_L,
             fused=False):
    """Inference forward of the 1-D SLA2 module (SLA2.forward without gradients,
    models/sla2_vendor/core.py:93-128), blockwise, CPU.

    Sparse branch: int8 -- _attn_fwd_int8 (models/sla2_vendor/kernel_sparse_qat.py:
    154-247): Q quantised per qblock rows (default bq), K and V per 64-row block,
    all with the round-half-away law of quantize_qkv; S = int(Q8 K8^T) (sq sk)
    scale log2(e), exact running maximum, P8 = trunc(127 P + 0.5), O += (P8 V8)
    sv / 127, o_s = O / l rounded to 16 bits.  Otherwise the 16-bit branch
    (_attn_fwd_qat without USE_INT8: O += round16(P) V).
    Linear branch: _hblocks and _lin_fwd3 (models/sla2_vendor/kernel_linear.py:
    396-493): kphi = round16(softmax_D(k)), HALL_j = round16(kphi_j^T V_j),
    ZALL_j = colsum kphi_j (fp32); H_i = sum_j HALL_j - sum_{j in lut_i} HALL_j,
    z_i likewise (fp32); num = qphi round16(H_i), den = qphi . z_i +- eps,
    o = round16(a o_s + (1 - a) o_l) with o_l = num / den, a fp32.

    fused: the arithmetic of the fused Algorithm-2 kernel instead
    (_sla2_fwd_fused, models/sla2_vendor/kernel_fused.py:29-124, Q scales per
    qblock = block_m rows): o_s stays fp32 (O / l, unrounded) into the mix,
    and the linear branch is the score form against the whole-sequence state,
    htot = round16(kphi^T V) over all L rows, ztot = colsum kphi (fp32),
    num = qphi htot - sum_{j in lut_i} round16(W_j) V_j,
    den = qphi . ztot - sum_j rowsum(W_j) +- eps, W_j = qphi kphi_j^T (fp32);
    o = round16(a o_s + (1 - a) num / den).  The caller averages alpha over
    heads, as the reference's SLA2.forward does for this kernel.

    q, k, v: (B,H,L,D) float tensors holding 16-bit values; alpha (H, ceil(L/bq))
    after the sigmoid; lut (B,H,ceil(L/bq),T).  Returns dict(o, o_s, lse, qphi,
    hall, zall).
    """
    B, H, L, D = q.shape
    nb = -(-L // E)
    lut64, a64 = _expand_1d(lut, alpha, bq, nb)               # per 64-row sub-block
    lut64 = torch.as_tensor(np.asarray(lut64)).long()
    T = lut64.shape[-1]
    if int8:
        qb = bq if qblock is None else qblock
        q8, qs_b = quantize_blocks(q, qb)
        k8, ks = quantize_blocks(k)
        v8, vs = quantize_blocks(v)
        qrow_s = torch.as_tensor(qs_b).float().repeat_interleave(qb, dim=-1)[..., :L]
    else:
        q8, k8, v8 = (torch.as_tensor(x).float().numpy() for x in (q, k, v))
        ks = vs = np.ones((B, H, nb), dtype=np.float32)
        qrow_s = torch.ones(B, H, L)
    qrow_s = torch.cat([qrow_s, qrow_s.new_ones(B, H, nb * E - L)], -1).view(B, H, nb, E)
    q8t = _tiles(torch.as_tensor(q8).double(), nb)
    k8t = _tiles(torch.as_tensor(k8).double(), nb)
    v8t = _tiles(torch.as_tensor(v8).double(), nb)
    ks, vs = torch.as_tensor(ks).float(), torch.as_tensor(vs).float()
    scale = float(np.float32(D ** -0.5))
    c2 = float(np.float32(scale * LOG2E))
    rows = torch.arange(nb * E).view(nb, E)
    m_i = torch.full((B, H, nb, E), -math.inf)
    l_i = torch.zeros(B, H, nb, E)
    o_s = torch.zeros(B, H, nb, E, D)
    for j in range(T):
        n = lut64[..., j]                                     # (B,H,nb)
        kt, vt = _gather_tiles(k8t, n), _gather_tiles(v8t, n)
        skn, svn = torch.gather(ks, 2, n), torch.gather(vs, 2, n)
        si = torch.matmul(q8t, kt.transpose(-1, -2)).float()  # exact integers (int8)
        if int8:
            qk = si * (qrow_s * skn[..., None])[..., None]
            qk = qk * c2
        else:
            qk = si * c2
        valid = rows[n] < L
        qk = qk.masked_fill(~valid[..., None, :], -math.inf)
        new_m = torch.maximum(m_i, qk.amax(-1))
        p = torch.exp2(qk - new_m[..., None])
        al = torch.exp2(m_i - new_m)
        o_s = o_s * al[..., None]
        if int8:
            p8 = torch.trunc(p * 127.0 + 0.5)
            o_s = o_s + torch.matmul(p8.double(), vt).float() * (svn / 127.0)[..., None, None]
        else:
            o_s = o_s + torch.matmul(_round16(p, t16).double(), vt).float()
        l_i = l_i * al + p.sum(-1)
        m_i = new_m
    o_s = (o_s / l_i[..., None]).reshape(B, H, nb * E, D)[:, :, :L]
    lse = (m_i + torch.log2(l_i)).reshape(B, H, nb * E)[:, :, :L]
    o_s16 = _round16(o_s, t16)
    qphi = _round16(torch.softmax(q.float(), -1), t16)
    kphi = _round16(torch.softmax(k.float(), -1), t16)
    kpt, vvt = _tiles(kphi, nb), _tiles(v.float(), nb)        # padding rows are zero
    hall = _round16(kpt.transpose(-1, -2) @ vvt, t16)          # (B,H,nb,D,D)
    zall = kpt.sum(-2)                                         # (B,H,nb,D)
    htot, ztot = hall.sum(2), zall.sum(2)
    lutq = torch.as_tensor(np.asarray(lut)).long()             # (B,H,Mq,T)
    Mq = lutq.shape[2]
    hsel = torch.stack([torch.stack([hall[b, h][lutq[b, h]].sum(1) for h in range(H)])
                        for b in range(B)])                    # (B,H,Mq,D,D)
    zsel = torch.stack([torch.stack([zall[b, h][lutq[b, h]].sum(1) for h in range(H)])
                        for b in range(B)])
    hi = htot[:, :, None] - hsel
    zi = ztot[:, :, None] - zsel
    qrow = torch.arange(L) // bq                               # query block of each row
    if fused:
        # kernel_fused.py:64-67, 108-114: per selected tile, in the score domain
        htot16 = _round16(kpt.reshape(B, H, nb * E, D).transpose(-1, -2)
                          @ vvt.reshape(B, H, nb * E, D), t16)           # (B,H,D,D)
        ztot = kpt.sum((2, 3))                                           # (B,H,D)
        num = qphi @ htot16
        den = (qphi * ztot[:, :, None, :]).sum(-1)
        lutr = lutq[:, :, qrow]                                          # (B,H,L,T)
        for j in range(lutq.shape[-1]):
            kp = torch.gather(kpt, 2, lutr[..., j].view(B, H, L, 1, 1).expand(B, H, L, E, D))
            vv = torch.gather(vvt, 2, lutr[..., j].view(B, H, L, 1, 1).expand(B, H, L, E, D))
            w = (qphi[..., None, :] * kp).sum(-1)                        # (B,H,L,E)
            num = num - (_round16(w, t16)[..., None] * vv).sum(-2)
            den = den - w.sum(-1)
        o_sm = o_s
    else:
        num = torch.einsum("bhld,bhlde->bhle", qphi, _round16(hi[:, :, qrow], t16))
        den = (qphi * zi[:, :, qrow]).sum(-1)
        o_sm = o_s16
    den = torch.where(den >= 0, den + eps, den - eps)
    o_l = num / den[..., None]
    a = torch.as_tensor(alpha).float()[:, qrow][None, :, :, None]
    o = _round16(a * o_sm + (1.0 - a) * o_l, t16)
    return {"o": o, "o_s": o_s16, "lse": lse, "qphi": qphi, "hall": hall, "zall": zall,
            "o_l": o_l}


def route_1d(q, k, topk_frac, bq, bk=E, proj_q=None, proj_k=None):
    """route_blocks with the canonical fp32 order (no smooth-k: the per-(b,h)
    key-mean shift adds a per-row constant to the scores).  Returns (lut, T)."""
    q, k = _np(q), _np(k)
    L, D = q.shape[-2:]
    mq, nb = -(-L // bq), -(-L // bk)
    qp = project_pool(pool_tiles(q, mq, L, block=bq), proj_q)
    kp = project_pool(pool_tiles(k, nb, L, block=bk), proj_k)
    pc = route_scores(qp, kp, D ** -0.5)
    T = topk_count(topk_frac, nb)
    return topk_rows(pc, T), T


def jvp_1d(q, k, v, dq, dk, dv, alpha, lut, bq, bk=E, t16=torch.float16, eps=EPS_L):
    """Blockwise restatement of sla2_mla_jvp (models/sla2_mla_jvp.py:348-385):
    _sla2_sparse_jvp_kernel (:108-197) over the routed key blocks -- 16-bit
    score operands, exact running maximum, P and T = P dS rounded to t16 for
    the P.V, T.V, P.dV products, l and mu from the unrounded P, T (products
    accumulated in fp32; the reference accumulates these dots in fp16) -- and
    _linear_jvp (:258-342): fp32 phi, per-key-block states, complement
    H_all - sum over the routed blocks, den + eps (unsigned), quotient rule;
    o = a o_s + (1-a) o_l per query block.  t16=None: no rounding (exact mode).
    Returns (o, do) fp32 (B,H,L,D)."""
    B, H, L, D = q.shape
    nb, mq = -(-L // bk), -(-L // bq)
    lut = torch.as_tensor(np.asarray(lut)).long()
    T = lut.shape[-1]
    dt = torch.float64 if t16 is None else torch.float32
    r16 = (lambda x: x) if t16 is None else (lambda x: x.to(t16).to(dt))
    f = lambda x: torch.as_tensor(x).to(dt)
    q, k, v, dq, dk, dv = (f(t) for t in (q, k, v, dq, dk, dv))
    scale = D ** -0.5
    c = scale * LOG2E if t16 is None else float(np.float32(np.float32(scale) * np.float32(LOG2E)))

    def qblocks(x):
        pad = mq * bq - L
        if pad:
            x = torch.cat([x, x.new_zeros(B, H, pad, x.shape[-1])], 2)
        return x.reshape(B, H, mq, bq, x.shape[-1])

    def kblocks(x):
        pad = nb * bk - L
        if pad:
            x = torch.cat([x, x.new_zeros(B, H, pad, x.shape[-1])], 2)
        return x.reshape(B, H, nb, bk, x.shape[-1])

    Qb, dQb = qblocks(q), qblocks(dq)
    Kb, dKb, Vb, dVb = kblocks(k), kblocks(dk), kblocks(v), kblocks(dv)
    gat = lambda xb, n: torch.gather(xb, 2, n.view(B, H, mq, 1, 1).expand(B, H, mq, bk, D))
    m_i = torch.full((B, H, mq, bq), -math.inf, dtype=dt)
    l_i = torch.zeros(B, H, mq, bq, dtype=dt)
    mu = torch.zeros(B, H, mq, bq, dtype=dt)
    acc_o = torch.zeros(B, H, mq, bq, D, dtype=dt)
    acc_do = torch.zeros(B, H, mq, bq, D, dtype=dt)
    key_pos = torch.arange(bk)
    for j in range(T):
        n = lut[..., j]
        kn, dkn, vn, dvn = gat(Kb, n), gat(dKb, n), gat(Vb, n), gat(dVb, n)
        s_f = Qb @ kn.transpose(-1, -2)
        ds = (dQb @ kn.transpose(-1, -2) + Qb @ dkn.transpose(-1, -2)) * scale
        valid = (n[..., None] * bk + key_pos) < L
        s2 = (s_f * c).masked_fill(~valid[..., None, :], -math.inf)
        m_new = torch.maximum(m_i, s2.amax(-1))
        al = torch.exp2(m_i - m_new)
        p = torch.exp2(s2 - m_new[..., None])
        t = p * ds
        l_i = l_i * al + p.sum(-1)
        mu = mu * al + t.sum(-1)
        pc, tc = r16(p), r16(t)
        acc_o = acc_o * al[..., None] + pc @ vn
        acc_do = acc_do * al[..., None] + tc @ vn + pc @ dvn
        m_i = m_new
    o_s = acc_o / l_i[..., None]
    do_s = acc_do / l_i[..., None] - (mu / l_i)[..., None] * o_s

    qphi, dqphi = phi_jvp(q, dq)
    kphi, dkphi = phi_jvp(k, dk)
    if t16 is None:
        qphi, dqphi, kphi, dkphi = (x.double() for x in (qphi, dqphi, kphi, dkphi))
    kb, dkb = kblocks(kphi), kblocks(dkphi)
    Hb = kb.transpose(-1, -2) @ Vb
    dHb = dkb.transpose(-1, -2) @ Vb + kb.transpose(-1, -2) @ dVb
    zb, dzb = kb.sum(3), dkb.sum(3)
    gat4 = lambda x: torch.gather(x, 2, lut.view(B, H, mq * T, 1, 1).expand(B, H, mq * T, D, D)
                                  ).view(B, H, mq, T, D, D).sum(3)
    gat3 = lambda x: torch.gather(x, 2, lut.view(B, H, mq * T, 1).expand(B, H, mq * T, D)
                                  ).view(B, H, mq, T, D).sum(3)
    Hc = Hb.sum(2)[:, :, None] - gat4(Hb)
    dHc = dHb.sum(2)[:, :, None] - gat4(dHb)
    zc = zb.sum(2)[:, :, None] - gat3(zb)
    dzc = dzb.sum(2)[:, :, None] - gat3(dzb)
    qg, dqg = qblocks(qphi), qblocks(dqphi)
    num = qg @ Hc
    dnum = dqg @ Hc + qg @ dHc
    den = (qg * zc[..., None, :]).sum(-1) + eps
    dden = (dqg * zc[..., None, :]).sum(-1) + (qg * dzc[..., None, :]).sum(-1)
    o_l = num / den[..., None]
    do_l = (dnum - o_l * dden[..., None]) / den[..., None]
    a = torch.as_tensor(alpha).to(dt).reshape(1, H, mq, 1, 1)
    o = a * o_s + (1.0 - a) * o_l
    do = a * do_s + (1.0 - a) * do_l
    return (o.reshape(B, H, mq * bq, D)[:, :, :L].float(),
            do.reshape(B, H, mq * bq, D)[:, :, :L].float())


def dense_1d_f64(q, k, v, lut, alpha, bq, bk=E, eps=EPS_L):
    """sla2_dense_ref (models/sla2_mla_jvp.py:388-418) in float64: masked softmax
    over the routed key blocks plus the complement linear branch, per-block alpha."""
    B, H, L, D = q.shape
    lut = torch.as_tensor(np.asarray(lut)).long()
    nb = -(-L // bk)
    mc = torch.zeros(B, H, lut.shape[2], nb, dtype=torch.float64)
    mc.scatter_(-1, lut, 1.0)
    m = mc.repeat_interleave(bq, dim=-2).repeat_interleave(bk, dim=-1)[..., :L, :L]
    s = (q @ k.transpose(-1, -2)) * D ** -0.5
    o_s = torch.softmax(s.masked_fill(m <= 0, -math.inf), dim=-1) @ v
    w = (torch.softmax(q, -1) @ torch.softmax(k, -1).transpose(-1, -2)) * (1.0 - m)
    o_l = (w @ v) / (w.sum(-1, keepdim=True) + eps)
    a = torch.as_tensor(alpha, dtype=torch.float64).repeat_interleave(bq, dim=-1)[:, :L]
    a = a.view(1, H, L, 1)
    return a * o_s + (1.0 - a) * o_l


# ---------------------------------------------------------------------------
# MLA attention sublayer and MLP sublayer JVP (models/mla_jvp_fast.py:53-228,
# kernels of models/triton_mla_block_jvp.py:237-498) and the eager block they
# differentiate (models/imf_dit_video.py:121-187, 266-284, 422-532).
# ---------------------------------------------------------------------------
def rms_jvp(x, dx, w, eps):
    """y = w x / r, dy = w (dx / r - x mean(x dx) / r^3), r = sqrt(mean(x^2) + eps)."""
    inv = 1.0 / torch.sqrt((x * x).mean(-1, keepdim=True) + eps)
    mxdx = (x * dx).mean(-1, keepdim=True)
    return w * x * inv, w * (dx * inv - x * (mxdx * inv ** 3))


def rope_rotate(x, cos, sin):
    """Rotate pairs (x[..., 2i], x[..., 2i+1]) of x (B, S, ..., 2*n) by (S, n) angles."""
    shape = (1, cos.shape[0]) + (1,) * (x.dim() - 3) + (cos.shape[1],)
    c, s = cos.reshape(shape), sin.reshape(shape)
    re, im = x[..., 0::2], x[..., 1::2]
    return torch.stack([re * c - im * s, re * s + im * c], -1).flatten(-2)


def mla_attn_jvp(h, dh, p, cos, sin, eps, attn_jvp, t16=torch.float16):
    """Hand-propagated JVP of a = out_proj(gate(attn(norm1(h)))) * g_attn with the
    reference fast path's 16-bit rounding points (stacked fp16 buffers, fp16
    weights, 16-bit GEMM outputs with fp32 accumulation); t16=None: exact.
    attn_jvp(q, k, v, dq, dk, dv) on (B, H, S, 64) in model order -> (o, do) fp32.
    Returns (a, da) (B, S, d)."""
    ex = t16 is None
    dt = torch.float64 if ex else torch.float32
    r = (lambda x: x) if ex else (lambda x: x.to(t16).to(dt))
    f = lambda x: torch.as_tensor(x).to(dt)
    h, dh = f(h), f(dh)
    B, S, D = h.shape
    H, dq, dc, dn, dr, dv = (p[n] for n in ("H", "dq", "dc", "dn", "dr", "dv"))
    W = lambda n: r(f(p[n]))
    lin = lambda x, w: r(x @ w.transpose(0, 1))
    n1, dn1 = (r(t) for t in rms_jvp(h, dh, f(p["w_norm1"]), eps))
    wa = torch.cat([W("w_qa"), W("w_kva")], 0)
    a_, da_ = lin(n1, wa), lin(dn1, wa)
    ql, dql = (r(t) for t in rms_jvp(a_[..., :dq], da_[..., :dq], f(p["w_qa_ln"]), eps))
    kl, dkl = (r(t) for t in rms_jvp(a_[..., dq:dq + dc], da_[..., dq:dq + dc],
                                     f(p["w_kva_ln"]), eps))
    qb = lin(ql, W("w_qb")).view(B, S, H, dn + dr)
    dqb = lin(dql, W("w_qb")).view(B, S, H, dn + dr)
    kvb = lin(kl, W("w_kvb")).view(B, S, H, dn + dv)
    dkvb = lin(dkl, W("w_kvb")).view(B, S, H, dn + dv)
    qn, dqn = rms_jvp(qb[..., :dn], dqb[..., :dn], f(p["w_qnorm"]), eps)
    kn, dkn = rms_jvp(kvb[..., :dn], dkvb[..., :dn], f(p["w_knorm"]), eps)
    c, s = f(cos), f(sin)
    qr, dqr = rope_rotate(qb[..., dn:], c, s), rope_rotate(dqb[..., dn:], c, s)
    kr = rope_rotate(a_[..., dq + dc:], c, s)[:, :, None].expand(B, S, H, dr)
    dkr = rope_rotate(da_[..., dq + dc:], c, s)[:, :, None].expand(B, S, H, dr)
    hd = lambda x: r(x).permute(0, 2, 1, 3).contiguous()
    q, dq_ = hd(torch.cat([qn, qr], -1)), hd(torch.cat([dqn, dqr], -1))
    k, dk = hd(torch.cat([kn, kr], -1)), hd(torch.cat([dkn, dkr], -1))
    v, dv_ = hd(kvb[..., dn:]), hd(dkvb[..., dn:])
    o, do = attn_jvp(q, k, v, dq_, dk, dv_)
    at = r(f(o).permute(0, 2, 1, 3).reshape(B, S, H * dv))
    dat = r(f(do).permute(0, 2, 1, 3).reshape(B, S, H * dv))
    if p.get("w_og") is not None:
        z, dz = lin(n1, W("w_og")), lin(dn1, W("w_og"))
        sg = torch.sigmoid(z)
        at, dat = r(at * sg), r(dat * sg + at * sg * (1 - sg) * dz)
    g = f(p["g_attn"])
    return lin(at, W("w_out")) * g, lin(dat, W("w_out")) * g


def mlp_jvp(h, dh, p, eps, t16=torch.float16):
    """Hand-propagated JVP of m = down(situ(gate_up(norm2(h)))) * g_mlp (the fast
    path has no linear_beta clamp of the up branch); t16=None: exact."""
    ex = t16 is None
    dt = torch.float64 if ex else torch.float32
    r = (lambda x: x) if ex else (lambda x: x.to(t16).to(dt))
    f = lambda x: torch.as_tensor(x).to(dt)
    h, dh = f(h), f(dh)
    lin = lambda x, w: r(x @ r(f(w)).transpose(0, 1))
    n2, dn2 = (r(t) for t in rms_jvp(h, dh, f(p["w_norm2"]), eps))
    wgu = torch.cat([f(p["w_gate"]), f(p["w_up"])], 0)
    gu, dgu = lin(n2, wgu), lin(dn2, wgu)
    F_ = gu.shape[-1] // 2
    g_, u, dg, du = gu[..., :F_], gu[..., F_:], dgu[..., :F_], dgu[..., F_:]
    beta = float(p.get("situ_beta", 1.0))
    sg, th = torch.sigmoid(g_), torch.tanh(g_ / beta)
    act = beta * th * sg
    dact = (1 - th * th) * sg + beta * th * sg * (1 - sg)
    hh, dhh = r(act * u), r(dact * dg * u + act * du)
    gm = f(p["g_mlp"])
    return lin(hh, p["w_down"]) * gm, lin(dhh, p["w_down"]) * gm


def mla_attn_eager(x, p, cos, sin, eps, attn):
    """MLAAttention.forward (models/imf_dit_video.py:422-467) applied to norm1(x)
    and times g_attn, in the dtype of x, with attn(q, k, v) on (B, H, S, 64)."""
    B, S, D = x.shape
    H, dq, dc, dn, dr, dv = (p[n] for n in ("H", "dq", "dc", "dn", "dr", "dv"))
    t = lambda n: torch.as_tensor(p[n]).to(x.dtype)
    rms = lambda y, w: w * y / torch.sqrt((y * y).mean(-1, keepdim=True) + eps)
    n1 = rms(x, t("w_norm1"))
    qb = (rms(n1 @ t("w_qa").T, t("w_qa_ln")) @ t("w_qb").T).view(B, S, H, dn + dr)
    kva = n1 @ t("w_kva").T
    kvb = (rms(kva[..., :dc], t("w_kva_ln")) @ t("w_kvb").T).view(B, S, H, dn + dv)
    c, s = torch.as_tensor(cos).to(x.dtype), torch.as_tensor(sin).to(x.dtype)
    q = torch.cat([rms(qb[..., :dn], t("w_qnorm")), rope_rotate(qb[..., dn:], c, s)], -1)
    kr = rope_rotate(kva[..., dc:], c, s)[:, :, None].expand(B, S, H, dr)
    k = torch.cat([rms(kvb[..., :dn], t("w_knorm")), kr], -1)
    v = kvb[..., dn:]
    o = attn(q.permute(0, 2, 1, 3), k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3))
    o = o.permute(0, 2, 1, 3).reshape(B, S, H * dv)
    if p.get("w_og") is not None:
        o = o * torch.sigmoid(n1 @ t("w_og").T)
    return (o @ t("w_out").T) * t("g_attn")


def mlp_eager(x, p, eps):
    """SwiGLUMlp(norm2(x)) * g_mlp without the linear_beta clamp."""
    t = lambda n: torch.as_tensor(p[n]).to(x.dtype)
    n2 = t("w_norm2") * x / torch.sqrt((x * x).mean(-1, keepdim=True) + eps)
    g_, u = n2 @ t("w_gate").T, n2 @ t("w_up").T
    beta = float(p.get("situ_beta", 1.0))
    return ((beta * torch.tanh(g_ / beta) * torch.sigmoid(g_) * u) @ t("w_down").T) * t("g_mlp")


def dense_attn_f64(q, k, v):
    """Softmax attention on (B, H, S, 64), scale 64^-0.5."""
    return torch.softmax((q @ k.transpose(-1, -2)) * q.shape[-1] ** -0.5, -1) @ v
