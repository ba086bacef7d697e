"""Torch-facing wrappers over the C ABI (include/sla2h.h).

Each function checks shapes and dtypes on the host, allocates its outputs
with torch's caching allocator on the inputs' device and launches on torch's
current HIP stream.  Inputs must already live on a GPU: there is no CPU path.
"""

import math

import torch

from . import _lib

E_TILE = 64
REC_BYTES = 2 * 16384 + 2 * 256  # sla2h_complement_record_bytes(64)


def _dtype_code(t):
    if t.dtype == torch.float16:
        return 0
    if t.dtype == torch.bfloat16:
        return 1
    raise TypeError(f"16-bit input expected (float16 / bfloat16), got {t.dtype}")


def _ptr(t):
    return None if t is None else ctypes_ptr(t)


def ctypes_ptr(t):
    return t.data_ptr()


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _need_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("sla2h ops run on the GPU only; got a tensor on " + str(t.device))


def _bhld(t, name):
    if t.dim() != 4 or t.shape[-1] != E_TILE:
        raise ValueError(f"{name}: expected (B, H, L, 64), got {tuple(t.shape)}")
    return t.contiguous()


def _check_lut(lut, B, H, L):
    Mb = -(-L // E_TILE)
    if lut.dim() != 4 or tuple(lut.shape[:3]) != (B, H, Mb):
        raise ValueError(f"lut: expected (B, H, Mb, T) = ({B}, {H}, {Mb}, T), got {tuple(lut.shape)}")


def check_lut_ids(lut, Np):
    """Raise ValueError unless every routed tile id of `lut` lies in [0, Np).

    The kernels take the ids as given (the fused kernel clamps them into range,
    the complement skips them), so a caller-supplied LUT holding -1 padding or
    a prefix-tail id would otherwise return wrong numbers.  One reduction and
    a device-to-host read: used on LUTs from outside, not on route_topk's."""
    if lut.numel() == 0:
        return
    lo, hi = int(lut.min().item()), int(lut.max().item())
    if lo < 0 or hi >= Np:
        raise ValueError(f"lut: tile ids must lie in [0, {Np}), got min {lo} max {hi}")


def _alpha_rows(alpha, H, Mb, device):
    """(H, Mb) fp32 with unit column stride (the kernels read alpha[h * stride + m])."""
    alpha = alpha.detach().to(device, torch.float32)
    if alpha.dim() != 2:
        alpha = alpha.reshape(H, -1)
    if tuple(alpha.shape) != (H, Mb):
        raise ValueError(f"alpha: expected (H, Mb) = ({H}, {Mb}), got {tuple(alpha.shape)}")
    return alpha if alpha.stride(1) == 1 else alpha.contiguous()


def quantize(x, E=E_TILE):
    """x (B,H,L,D) 16-bit -> (xq int8 (B,H,L,D), xs fp32 (B,H,ceil(L/E)))."""
    _need_gpu(x)
    x = _bhld(x, "x")
    B, H, L, D = x.shape
    nb = -(-L // E)
    xq = torch.empty_like(x, dtype=torch.int8)
    xs = torch.empty(B, H, nb, device=x.device, dtype=torch.float32)
    _lib.check(_lib.load().sla2h_quantize(x.data_ptr(), _dtype_code(x), B * H, L, D, E,
                                          xq.data_ptr(), xs.data_ptr(), _stream(x.device)),
               "sla2h_quantize")
    return xq, xs


def quant_pool_qk(q, k, Np, E=E_TILE, proj_q=None, proj_k=None, with_kb=False):
    """INT8 Q/K with per-block scales plus the router's pooled (projected) tiles.

    Returns q8, qs, k8, ks, qpool (B,H,Nb,D) fp32, kpool_t (B,H,D,Np) fp32,
    and with with_kb also kb (B,H,Nb) fp32: per key block a bound on
    max ||k8_j|| * ks over its rows (the static softmax shift of fwd_jvp).
    """
    _need_gpu(q, k)
    q, k = _bhld(q, "q"), _bhld(k, "k")
    if q.shape != k.shape or q.dtype != k.dtype:
        raise ValueError("q and k must share shape and dtype")
    B, H, L, D = q.shape
    nb = -(-L // E)
    dev = q.device
    pq = None if proj_q is None else proj_q.detach().to(dev, torch.float32).contiguous()
    pk = None if proj_k is None else proj_k.detach().to(dev, torch.float32).contiguous()
    q8 = torch.empty_like(q, dtype=torch.int8)
    k8 = torch.empty_like(k, dtype=torch.int8)
    qs = torch.empty(B, H, nb, device=dev, dtype=torch.float32)
    ks = torch.empty_like(qs)
    qpool = torch.empty(B, H, nb, D, device=dev, dtype=torch.float32)
    kpool_t = torch.empty(B, H, D, Np, device=dev, dtype=torch.float32)
    kb = torch.empty(B, H, nb, device=dev, dtype=torch.float32) if with_kb else None
    _lib.check(_lib.load().sla2h_quant_pool_qk(
        q.data_ptr(), k.data_ptr(), _dtype_code(q), B, H, L, D, E, Np,
        _ptr(pq), _ptr(pk), q8.data_ptr(), qs.data_ptr(), k8.data_ptr(), ks.data_ptr(),
        qpool.data_ptr(), kpool_t.data_ptr(), _ptr(kb), _stream(dev)), "sla2h_quant_pool_qk")
    if with_kb:
        return q8, qs, k8, ks, qpool, kpool_t, kb
    return q8, qs, k8, ks, qpool, kpool_t


def topk_count(topk_frac, Np):
    """T = max(1, min(Np, int(frac * Np))) (models/mla_video_sparse_jvp.py:564)."""
    return max(1, min(Np, int(topk_frac * Np)))


def route_topk(qpool, kpool_t, T, scale, with_mask=False):
    """Top-T key tiles per query block -> lut (B,H,Mb,T) int32 [, mask (B,H,Mb,Np) uint8]."""
    _need_gpu(qpool, kpool_t)
    B, H, Mb, D = qpool.shape
    Np = kpool_t.shape[-1]
    lut = torch.empty(B, H, Mb, T, device=qpool.device, dtype=torch.int32)
    mask = (torch.empty(B, H, Mb, Np, device=qpool.device, dtype=torch.uint8)
            if with_mask else None)
    _lib.check(_lib.load().sla2h_route_topk(
        qpool.contiguous().data_ptr(), kpool_t.contiguous().data_ptr(), B, H, Mb, Np, D, T,
        float(scale), lut.data_ptr(), _ptr(mask), _stream(qpool.device)), "sla2h_route_topk")
    return (lut, mask) if with_mask else lut


def linear_states(k, v, Np, dk=None, dv=None, E=E_TILE, with_sums=True):
    """phi(K)-states of the video tiles, their sums and the value-operand tiles.

    Returns a dict with Hb, zb, vt [, Hall, zall] (and dHb, dzb [, dHall,
    dzall] when dk/dv are given; vt then interleaves V and dV).  The sums over
    the tiles are skipped with with_sums=False (the fused op does not need them).
    """
    _need_gpu(k, v, dk, dv)
    k, v = _bhld(k, "k"), _bhld(v, "v")
    tan = dk is not None
    if tan:
        dk, dv = _bhld(dk, "dk"), _bhld(dv, "dv")
    B, H, L, D = k.shape
    nb = -(-L // E)
    dev, f32 = k.device, torch.float32
    st = {
        "Hb": torch.empty(B, H, Np, D, D, device=dev, dtype=f32),
        "zb": torch.empty(B, H, Np, D, device=dev, dtype=f32),
        "vt": torch.empty(B, H, nb, D, E * (2 if tan else 1), device=dev, dtype=v.dtype),
    }
    if tan:
        st.update({"dHb": torch.empty_like(st["Hb"]), "dzb": torch.empty_like(st["zb"]),
                   "kt": torch.empty(B, H, nb, D, 2 * E, device=dev, dtype=k.dtype)})
    if with_sums:
        st.update({"Hall": torch.empty(B, H, D, D, device=dev, dtype=f32),
                   "zall": torch.empty(B, H, D, device=dev, dtype=f32)})
        if tan:
            st.update({"dHall": torch.empty_like(st["Hall"]),
                       "dzall": torch.empty_like(st["zall"])})
    g = lambda n: _ptr(st.get(n))
    _lib.check(_lib.load().sla2h_linear_states(
        k.data_ptr(), _ptr(dk), v.data_ptr(), _ptr(dv), _dtype_code(k), B, H, L, D, E, Np,
        g("Hb"), g("dHb"), g("zb"), g("dzb"), g("Hall"), g("dHall"), g("zall"), g("dzall"),
        g("vt"), g("kt"), _stream(dev)), "sla2h_linear_states")
    return st


COMPLEMENT_SCRATCH_BYTES = 4 << 20  # SLA2H_COMPLEMENT_SCRATCH_BYTES


def complement(st, lut, Np, noalloc=False, check_ids=True):
    """Per-query-block complement records (uint8 (B,H,Mb,REC_BYTES)).

    noalloc: run sla2h_complement_noalloc, whose bit-mask workspace is the
    library's static per-GPU array (at most COMPLEMENT_SCRATCH_BYTES) instead
    of a torch allocation; concurrent calls on one GPU must not overlap.
    check_ids: validate the LUT's tile ids (check_lut_ids); False for a LUT
    straight from route_topk."""
    B, H, Mb, T = lut.shape
    if check_ids:
        check_lut_ids(lut, Np)
    lib = _lib.load()
    comp = torch.empty(B, H, Mb, REC_BYTES, device=lut.device, dtype=torch.uint8)
    g = lambda n: _ptr(st.get(n))
    need = lib.sla2h_complement_workspace_bytes(B, H, Mb, Np)
    if noalloc:
        if need > COMPLEMENT_SCRATCH_BYTES:
            raise ValueError(f"complement(noalloc=True): the bit masks need {need} bytes, over "
                             f"the static {COMPLEMENT_SCRATCH_BYTES}-byte array")
        with torch.cuda.device(lut.device):
            _lib.check(lib.sla2h_complement_noalloc(
                g("Hb"), g("dHb"), g("zb"), g("dzb"), lut.contiguous().data_ptr(), B, H, Mb,
                Np, E_TILE, T, comp.data_ptr(), _stream(lut.device)), "sla2h_complement_noalloc")
        return comp
    ws = torch.empty(need, device=lut.device, dtype=torch.uint8)
    _lib.check(lib.sla2h_complement(
        g("Hb"), g("dHb"), g("zb"), g("dzb"), lut.contiguous().data_ptr(), B, H, Mb, Np,
        E_TILE, T, ws.data_ptr(), comp.data_ptr(), _stream(lut.device)), "sla2h_complement")
    return comp


def fwd_jvp(q, q8, k8, qs, ks, st, comp, alpha, lut, Np, dq=None, scale=None, eps_l=1e-5,
            sparse_only=False, kb=None, check_ids=True):
    """The fused sparse+linear op (and JVP when dq is given) -> (o, do|None) fp32.

    The key side comes from k8/ks and the operand tiles of `st`
    (linear_states with tangents when dq is given).  kb (quant_pool_qk's
    with_kb output) enables the static softmax shift; None keeps the running
    maximum everywhere.  check_ids validates the LUT's tile ids
    (check_lut_ids); False for a LUT straight from route_topk.
    """
    _need_gpu(q, dq, alpha, lut)
    if check_ids:
        check_lut_ids(lut, Np)
    B, H, L, D = q.shape
    T = lut.shape[-1]
    tan = dq is not None
    if tan != ("dHb" in st):
        raise ValueError("fwd_jvp: the states must be built with tangents exactly when dq is given")
    scale = D ** -0.5 if scale is None else scale
    o = torch.empty(B, H, L, D, device=q.device, dtype=torch.float32)
    do = torch.empty_like(o) if tan else None
    _check_lut(lut, B, H, L)
    if alpha is not None:
        alpha = _alpha_rows(alpha, H, -(-L // E_TILE), q.device)
    _lib.check(_lib.load().sla2h_fwd_jvp(
        q.data_ptr(), _ptr(dq), _ptr(st.get("kt")) if tan else None, st["vt"].data_ptr(),
        q8.data_ptr(), k8.data_ptr(), qs.data_ptr(),
        ks.data_ptr(), _ptr(kb), _ptr(comp), _ptr(alpha), 0 if alpha is None else alpha.stride(0),
        lut.contiguous().data_ptr(), _dtype_code(q), B, H, L, D, E_TILE, Np, T, float(scale),
        float(eps_l), 1 if sparse_only else 0, o.data_ptr(), _ptr(do), _stream(q.device)),
        "sla2h_fwd_jvp")
    return o, do


def cube_jvp(q, k, v, dq, dk, dv, alpha, topk_frac, Np, prefix_len=0, proj_q=None,
             proj_k=None, lut=None, T=None, return_aux=False):
    """Whole fused op: quant+pool, route (unless lut given), states, complement, attention.

    q..dv: (B,H,L,64) 16-bit, tile-major; dq/dk/dv None = primal only.
    alpha: (H, Mb) after the sigmoid.  Returns (o, do) fp32 (do None if primal).
    """
    B, H, L, D = q.shape
    E = E_TILE
    nb = -(-L // E)
    if nb != Np + (-(-prefix_len // E) if prefix_len else 0):
        raise ValueError(f"L={L} does not match Np={Np}, E={E}, prefix_len={prefix_len}")
    q, k, v = (t.contiguous() for t in (q, k, v))
    tan = dq is not None
    if tan:
        dq, dk, dv = (t.to(q.dtype).contiguous() for t in (dq, dk, dv))
    q8, qs, k8, ks, qpool, kpool_t, kb = quant_pool_qk(q, k, Np, E, proj_q, proj_k, with_kb=True)
    if lut is None:
        T = topk_count(topk_frac, Np)
        lut = route_topk(qpool, kpool_t, T, D ** -0.5)
    else:
        lut = lut.to(torch.int32).contiguous()
        T = lut.shape[-1]
        check_lut_ids(lut, Np)
    st = linear_states(k, v, Np, dk if tan else None, dv if tan else None, E, with_sums=False)
    comp = complement(st, lut, Np, check_ids=False)
    o, do = fwd_jvp(q, q8, k8, qs, ks, st, comp, alpha, lut, Np, dq if tan else None, kb=kb,
                    check_ids=False)
    if return_aux:
        aux = dict(q8=q8, qs=qs, k8=k8, ks=ks, kb=kb, qpool=qpool, kpool_t=kpool_t, lut=lut, T=T,
                   comp=comp, **st)
        return o, do, aux
    return o, do


# ---------------------------------------------------------------------------
# Training forward (_CubeQATFunction.forward, models/sla2_cube_qat.py:703-752)
# ---------------------------------------------------------------------------

def quant_train(q, k, v, E=E_TILE):
    """Truncating INT8 quantisation of Q, K, V (the training kernel's law).

    -> dict(q8, qs, k8, ks, v8f, vs); v8f (B,H,Nb,4096) int8 in fragment order.
    """
    _need_gpu(q, k, v)
    q, k, v = (_bhld(t, n) for t, n in ((q, "q"), (k, "k"), (v, "v")))
    if not (q.shape == k.shape == v.shape and q.dtype == k.dtype == v.dtype):
        raise ValueError("quant_train: q, k, v must share shape and dtype")
    B, H, L, D = q.shape
    nb = -(-L // E)
    dev = q.device
    out = dict(q8=torch.empty_like(q, dtype=torch.int8), k8=torch.empty_like(k, dtype=torch.int8),
               v8f=torch.empty(B, H, nb, 4096, device=dev, dtype=torch.int8))
    for n in ("qs", "ks", "vs"):
        out[n] = torch.empty(B, H, nb, device=dev, dtype=torch.float32)
    _lib.check(_lib.load().sla2h_quant_train(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _dtype_code(q), B, H, L, D, E,
        out["q8"].data_ptr(), out["qs"].data_ptr(), out["k8"].data_ptr(), out["ks"].data_ptr(),
        out["v8f"].data_ptr(), out["vs"].data_ptr(), _stream(dev)), "sla2h_quant_train")
    return out


def sparse_fwd_qat(q, qz, lut, Np, scale=None):
    """Sparse branch of the training forward -> (o_s 16-bit, lse fp32, qphi 16-bit)."""
    _need_gpu(q, lut)
    B, H, L, D = q.shape
    T = lut.shape[-1]
    _check_lut(lut, B, H, L)
    scale = D ** -0.5 if scale is None else scale
    o_s = torch.empty_like(q)
    qphi = torch.empty_like(q)
    lse = torch.empty(B, H, L, device=q.device, dtype=torch.float32)
    _lib.check(_lib.load().sla2h_sparse_fwd_qat(
        q.data_ptr(), qz["q8"].data_ptr(), qz["qs"].data_ptr(), qz["k8"].data_ptr(),
        qz["ks"].data_ptr(), qz["v8f"].data_ptr(), qz["vs"].data_ptr(),
        lut.to(torch.int32).contiguous().data_ptr(), _dtype_code(q), B, H, L, D, E_TILE, Np, T,
        float(scale), o_s.data_ptr(), lse.data_ptr(), qphi.data_ptr(), _stream(q.device)),
        "sla2h_sparse_fwd_qat")
    return o_s, lse, qphi


def linear_states_qat(k, v, with_vt=False):
    """States of all Nb tiles with 16-bit-rounded phi(K) -> dict(Hb, zb, Hall, zall[, vt])."""
    _need_gpu(k, v)
    k, v = _bhld(k, "k"), _bhld(v, "v")
    B, H, L, D = k.shape
    nb = -(-L // E_TILE)
    dev = k.device
    st = dict(Hb=torch.empty(B, H, nb, D, D, device=dev), zb=torch.empty(B, H, nb, D, device=dev),
              Hall=torch.empty(B, H, D, D, device=dev), zall=torch.empty(B, H, D, device=dev))
    if with_vt:
        st["vt"] = torch.empty(B, H, nb, D, E_TILE, device=dev, dtype=v.dtype)
    _lib.check(_lib.load().sla2h_linear_states_qat(
        k.data_ptr(), v.data_ptr(), _dtype_code(k), B, H, L, D, E_TILE, st["Hb"].data_ptr(),
        st["zb"].data_ptr(), st["Hall"].data_ptr(), st["zall"].data_ptr(), _ptr(st.get("vt")),
        _stream(dev)), "sla2h_linear_states_qat")
    return st


def linear_mix_qat(qphi, comp, Hall, o_s, alpha, eps_l=1e-5, bq=E_TILE):
    """Linear branch + alpha mix of the training forward -> (o, o_l 16-bit, den fp32).
    comp and alpha are per query block of bq rows."""
    _need_gpu(qphi, comp, Hall, o_s, alpha)
    B, H, L, D = qphi.shape
    Mq = -(-L // bq)
    if tuple(comp.shape) != (B, H, Mq, REC_BYTES) or tuple(Hall.shape) != (B, H, D, D):
        raise ValueError("linear_mix_qat: comp / Hall shapes do not match qphi")
    alpha = _alpha_rows(alpha, H, Mq, qphi.device)
    o = torch.empty_like(o_s)
    o_l = torch.empty_like(o_s)
    den = torch.empty(B, H, L, device=qphi.device, dtype=torch.float32)
    _lib.check(_lib.load().sla2h_linear_mix_qat(
        qphi.data_ptr(), comp.data_ptr(), Hall.contiguous().data_ptr(), o_s.data_ptr(),
        alpha.data_ptr(), alpha.stride(0), _dtype_code(qphi), B, H, L, D, bq,
        float(eps_l), o.data_ptr(), o_l.data_ptr(), den.data_ptr(), _stream(qphi.device)),
        "sla2h_linear_mix_qat")
    return o, o_l, den


SCORE_FORM_MAX_J = 4


def linear_mix_score(qphi, k, v, st, lut, o_s, alpha, eps_l=1e-5, bq=E_TILE):
    """Score form of linear_mix_qat (the reference's branch for LUTs of at most
    SCORE_FORM_MAX_J columns): the routed tiles are subtracted as
    round16(qphi kphi_j^T) v_j from qphi round16(Hall), not from the state.
    st: linear_states_qat's dict (Hall, zall); lut (B,H,ceil(L/bq),J) int32,
    ids in [0, ceil(L/64)).  Returns (o, o_l 16-bit, den fp32)."""
    _need_gpu(qphi, k, v, lut, o_s, alpha)
    B, H, L, D = qphi.shape
    Mq = -(-L // bq)
    lut = lut.to(torch.int32).contiguous()
    if lut.dim() != 4 or tuple(lut.shape[:3]) != (B, H, Mq):
        raise ValueError(f"linear_mix_score: lut must be (B, H, {Mq}, J), got {tuple(lut.shape)}")
    for t in (k, v, o_s):
        if tuple(t.shape) != (B, H, L, D) or t.dtype != qphi.dtype:
            raise ValueError("linear_mix_score: k, v, o_s must match qphi")
    alpha = _alpha_rows(alpha, H, Mq, qphi.device)
    o = torch.empty_like(o_s)
    o_l = torch.empty_like(o_s)
    den = torch.empty(B, H, L, device=qphi.device, dtype=torch.float32)
    _lib.check(_lib.load().sla2h_linear_mix_score(
        qphi.data_ptr(), k.contiguous().data_ptr(), v.contiguous().data_ptr(),
        st["Hall"].contiguous().data_ptr(), st["zall"].contiguous().data_ptr(), lut.data_ptr(),
        lut.shape[-1], o_s.data_ptr(), alpha.data_ptr(), alpha.stride(0), _dtype_code(qphi),
        B, H, L, D, bq, float(eps_l), o.data_ptr(), o_l.data_ptr(), den.data_ptr(),
        _stream(qphi.device)), "sla2h_linear_mix_score")
    return o, o_l, den


def augment_lut(lut, Np, n_tail):
    """lut (B,H,Mb,T) -> lut_aug (B,H,Mb,T+n_tail) int32 with the prefix tail blocks appended."""
    B, H, Mb, _ = lut.shape
    tail = torch.arange(Np, Np + n_tail, device=lut.device, dtype=torch.int32)
    return torch.cat([lut.to(torch.int32), tail.view(1, 1, 1, -1).expand(B, H, Mb, n_tail)],
                     -1).contiguous()


def train_fwd(q, k, v, alpha, lut, Np, eps_l=1e-5, int8=True):
    """Training forward of the cube-QAT op on given routing.

    q, k, v: (B,H,L,64) 16-bit, tile-major.  alpha: (H, Mb) after the sigmoid.
    lut: (B,H,Mb,T) routed video tiles.  int8: the INT8 sparse branch of
    _attn_fwd_qat (truncating Q/K/V quantisation, INT8 P.V), else its 16-bit
    branch (S = q.k^T on 16-bit MFMA, O += round16(P).V), as the reference
    module's use_int8 flag selects (models/sla2_cube_qat.py:395, 413).  The
    linear branch runs in the score form while the augmented LUT has at most
    SCORE_FORM_MAX_J columns, else in the state form (models/sla2_cube_qat.py:739).
    Returns a dict with the module output o and the tensors the reference
    saves for its backward: o_s, o_l, lse, den, qphi, htot (rounded to 16
    bits, held in fp32), ztot, lut_aug, and (int8) the quantised operands.
    """
    q, k, v = (t.contiguous() for t in (q, k, v))
    B, H, L, D = q.shape
    nb = -(-L // E_TILE)
    n_tail = nb - Np
    lut = lut.to(torch.int32).contiguous()
    lut_aug = augment_lut(lut, Np, n_tail)
    qz = {}
    if int8:
        qz = quant_train(q, k, v)
        o_s, lse, qphi = sparse_fwd_qat(q, qz, lut, Np)
        st = linear_states_qat(k, v)
    else:
        st = linear_states_qat(k, v, with_vt=True)
        o_s, lse, qphi = sparse_fwd_16(q, k, st["vt"], lut_aug, E_TILE)
    # the complement records also feed the backward's dqphi
    comp = complement(st, lut_aug, nb, check_ids=False)
    if lut_aug.shape[-1] <= SCORE_FORM_MAX_J:
        o, o_l, den = linear_mix_score(qphi, k, v, st, lut_aug, o_s, alpha, eps_l)
    else:
        o, o_l, den = linear_mix_qat(qphi, comp, st["Hall"], o_s, alpha, eps_l)
    htot = st["Hall"].to(q.dtype).float()
    return dict(o=o, o_s=o_s, o_l=o_l, lse=lse, den=den, qphi=qphi, htot=htot,
                ztot=st["zall"], Hall=st["Hall"], comp=comp, lut_aug=lut_aug, **qz)


def train_bwd(q, k, v, alpha, fwd, do, scale=None, stage_events=None, bq=E_TILE):
    """Straight-through backward of train_fwd (bq = 64) or train_fwd_1d.

    q, k, v: the forward's 16-bit inputs; alpha (H, Mq) after the sigmoid, one
    column per query block of bq rows; fwd: the forward's dict; do: (B,H,L,D)
    output gradient.  Returns (dq, dk, dv) 16-bit and d_alpha (H, Mq) fp32,
    the gradient with respect to the alpha logits.
    """
    _need_gpu(q, k, v, do)
    q, k, v = (t.contiguous() for t in (q, k, v))
    B, H, L, D = q.shape
    nb = -(-L // E_TILE)
    dev = q.device
    scale = D ** -0.5 if scale is None else scale
    do = do.to(q.dtype).contiguous()
    mq = -(-L // bq)
    alpha = _alpha_rows(alpha, H, mq, dev)
    lib = _lib.load()
    f16 = lambda: torch.empty_like(q)
    dos, g16 = f16(), f16()
    delta = torch.empty(B, H, L, device=dev)
    srow = torch.empty(B, H, L, device=dev)
    seg = torch.zeros(H, mq, device=dev)
    P = torch.empty(B, H, nb, D, D, device=dev)
    Pz = torch.empty(B, H, nb, D, device=dev)
    dc = _dtype_code(q)
    st = _stream(dev)
    rec = (lambda i: stage_events[i].record()) if stage_events else (lambda i: None)
    rec(0)
    _lib.check(lib.sla2h_bwd_prep(
        do.data_ptr(), fwd["o_s"].data_ptr(), fwd["o_l"].data_ptr(), fwd["den"].data_ptr(),
        fwd["qphi"].data_ptr(), alpha.data_ptr(), alpha.stride(0), dc, B, H, L, D, bq,
        dos.data_ptr(), delta.data_ptr(), g16.data_ptr(), srow.data_ptr(), seg.data_ptr(),
        P.data_ptr(), Pz.data_ptr(), st), "sla2h_bwd_prep")
    lut_aug = fwd["lut_aug"]
    J = lut_aug.shape[-1]
    ncq = -(-nb // 32)
    sel = torch.empty(B, H, nb, ncq, device=dev, dtype=torch.int32)
    ws = torch.empty(lib.sla2h_complement_workspace_bytes(B, H, nb, nb), device=dev,
                     dtype=torch.uint8)
    compb = torch.empty(B, H, nb, REC_BYTES, device=dev, dtype=torch.uint8)
    rec(1)
    _lib.check(lib.sla2h_complement_bwd(P.data_ptr(), Pz.data_ptr(), lut_aug.data_ptr(), B, H,
                                        nb, bq, J, ws.data_ptr(), sel.data_ptr(),
                                        compb.data_ptr(), st), "sla2h_complement_bwd")
    dq, dk, dv = f16(), f16(), f16()
    rec(2)
    _lib.check(lib.sla2h_bwd_dq(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), dos.data_ptr(), fwd["lse"].data_ptr(),
        delta.data_ptr(), g16.data_ptr(), srow.data_ptr(), fwd["comp"].data_ptr(),
        fwd["Hall"].data_ptr(), fwd["qphi"].data_ptr(), lut_aug.data_ptr(), dc, B, H, L, D, bq,
        J, float(scale), dq.data_ptr(), st), "sla2h_bwd_dq")
    rec(3)
    _lib.check(lib.sla2h_bwd_dkdv(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), dos.data_ptr(), fwd["lse"].data_ptr(),
        delta.data_ptr(), sel.data_ptr(), compb.data_ptr(), dc,
        B, H, L, D, E_TILE, float(scale), dk.data_ptr(), dv.data_ptr(), st), "sla2h_bwd_dkdv")
    d_alpha = seg * alpha * (1.0 - alpha)
    return dq, dk, dv, d_alpha


# ---------------------------------------------------------------------------
# 1-D SLA2 blocks: query blocks of bq rows, key blocks of 64 rows
# ---------------------------------------------------------------------------

def pool_blocks(x, blk, proj=None, transposed=False):
    """Block means of x (B,H,L,64) 16-bit or fp32 over blk rows (+ projection)
    -> fp32 (B,H,nblk,64), or (B,H,64,nblk) when transposed."""
    _need_gpu(x, proj)
    x = _bhld(x, "x")
    B, H, L, D = x.shape
    nblk = -(-L // blk)
    shape = (B, H, D, nblk) if transposed else (B, H, nblk, D)
    out = torch.empty(shape, device=x.device, dtype=torch.float32)
    if proj is not None:
        proj = proj.detach().to(x.device, torch.float32).contiguous()
    code = 2 if x.dtype == torch.float32 else _dtype_code(x)
    _lib.check(_lib.load().sla2h_pool_blocks(
        x.data_ptr(), code, B * H, L, D, blk, _ptr(proj), 1 if transposed else 0,
        out.data_ptr(), _stream(x.device)), "sla2h_pool_blocks")
    return out


def route_1d(q, k, topk_frac, bq, bk=E_TILE, proj_q=None, proj_k=None):
    """1-D router: pooled-score hard top-k -> (lut (B,H,ceil(L/bq),T) int32, T)."""
    if bk != E_TILE:
        raise ValueError(f"key blocks must be {E_TILE} rows, got {bk}")
    B, H, L, D = q.shape
    nb = -(-L // bk)
    T = max(1, min(nb, int(topk_frac * nb)))
    qpool = pool_blocks(q, bq, proj_q)
    kpool_t = pool_blocks(k, bk, proj_k, transposed=True)
    return route_topk(qpool, kpool_t, T, D ** -0.5), T


def jvp_1d(q, k, v, dq, dk, dv, alpha, lut, bq, scale=None, eps_l=1e-5, return_aux=False):
    """1-D SLA2 attention and its JVP on given routing -> (o, do) fp32."""
    _need_gpu(q, k, v, dq, dk, dv, lut)
    q, k, v, dq, dk, dv = (_bhld(t, "qkv") for t in (q, k, v, dq, dk, dv))
    B, H, L, D = q.shape
    nb = -(-L // E_TILE)
    mq = -(-L // bq)
    lut = lut.to(torch.int32).contiguous()
    if lut.dim() != 4 or tuple(lut.shape[:3]) != (B, H, mq):
        raise ValueError(f"lut: expected (B, H, {mq}, T), got {tuple(lut.shape)}")
    T = lut.shape[-1]
    alpha = _alpha_rows(alpha, H, mq, q.device)
    scale = D ** -0.5 if scale is None else scale
    st = linear_states(k, v, nb, dk, dv, with_sums=False)
    comp = complement(st, lut, nb, check_ids=False)
    o = torch.empty(B, H, L, D, device=q.device, dtype=torch.float32)
    do = torch.empty_like(o)
    _lib.check(_lib.load().sla2h_fwd_jvp_1d(
        q.data_ptr(), dq.data_ptr(), st["kt"].data_ptr(), st["vt"].data_ptr(), comp.data_ptr(),
        alpha.data_ptr(), alpha.stride(0), lut.data_ptr(), _dtype_code(q), B, H, L, D, bq,
        E_TILE, T, float(scale), float(eps_l), o.data_ptr(), do.data_ptr(), _stream(q.device)),
        "sla2h_fwd_jvp_1d")
    if return_aux:
        return o, do, dict(comp=comp, **st)
    return o, do


def sparse_fwd_16(q, k, vt, lut, bq, scale=None):
    """16-bit sparse branch of _attn_fwd_qat (no USE_INT8) over the routed
    64-row key blocks of lut (B,H,ceil(L/bq),J): S = q.k^T on 16-bit MFMA,
    exact running maximum, O += round16(P).V with V from the primal operand
    tiles vt of linear_states_qat / hblocks_states.  Any routed block may be
    the partial last one.  -> (o_s 16-bit, lse fp32 log2 domain, qphi 16-bit)."""
    _need_gpu(q, k, vt, lut)
    B, H, L, D = q.shape
    mq = -(-L // bq)
    lut = lut.to(torch.int32).contiguous()
    if lut.dim() != 4 or tuple(lut.shape[:3]) != (B, H, mq):
        raise ValueError(f"lut: expected (B, H, {mq}, J), got {tuple(lut.shape)}")
    scale = D ** -0.5 if scale is None else scale
    o_s, qphi = torch.empty_like(q), torch.empty_like(q)
    lse = torch.empty(B, H, L, device=q.device, dtype=torch.float32)
    _lib.check(_lib.load().sla2h_sparse_fwd_1d(
        q.data_ptr(), k.data_ptr(), vt.data_ptr(), lut.data_ptr(), _dtype_code(q), B, H, L, D,
        bq, E_TILE, lut.shape[-1], float(scale), o_s.data_ptr(), lse.data_ptr(),
        qphi.data_ptr(), _stream(q.device)), "sla2h_sparse_fwd_1d")
    return o_s, lse, qphi


def cube_jvp16(q, k, v, dq, dk, dv, alpha, lut, Np, scale=None, eps_l=1e-5):
    """Cube-tile SLA2 JVP with 16-bit primal scores (the reference's non-QAT
    mla_video_sparse_jvp, models/mla_video_sparse_jvp.py:403-454): the sparse
    branch visits the routed video tiles of lut (B,H,Mb,T) and every prefix
    tail block, the linear branch the complement over the Np video tiles, then
    the alpha mix.  q..dv (B,H,L,64) 16-bit tile-major; alpha (H, Mb).
    -> (o, do) fp32."""
    _need_gpu(q, k, v, dq, dk, dv, lut)
    q, k, v, dq, dk, dv = (_bhld(t, "qkv") for t in (q, k, v, dq, dk, dv))
    B, H, L, D = q.shape
    nb = -(-L // E_TILE)
    lut = lut.to(torch.int32).contiguous()
    _check_lut(lut, B, H, L)
    alpha = _alpha_rows(alpha, H, nb, q.device)
    scale = D ** -0.5 if scale is None else scale
    st = linear_states(k, v, Np, dk, dv, with_sums=False)
    comp = complement(st, lut, Np, check_ids=False)
    lut_aug = augment_lut(lut, Np, nb - Np)
    o = torch.empty(B, H, L, D, device=q.device, dtype=torch.float32)
    do = torch.empty_like(o)
    _lib.check(_lib.load().sla2h_fwd_jvp_1d(
        q.data_ptr(), dq.data_ptr(), st["kt"].data_ptr(), st["vt"].data_ptr(), comp.data_ptr(),
        alpha.data_ptr(), alpha.stride(0), lut_aug.data_ptr(), _dtype_code(q), B, H, L, D,
        E_TILE, E_TILE, lut_aug.shape[-1], float(scale), float(eps_l), o.data_ptr(),
        do.data_ptr(), _stream(q.device)), "sla2h_fwd_jvp_1d")
    return o, do


def train_fwd_1d(q, k, v, alpha, lut, bq, eps_l=1e-5, int8=False):
    """Training forward of the 1-D SLA2 module on given routing.

    q, k, v: (B,H,L,64) 16-bit, natural order.  alpha (H, ceil(L/bq)) after the
    sigmoid; lut (B,H,ceil(L/bq),T) routed 64-row key blocks.  int8: the INT8
    sparse branch of _attn_fwd_qat (truncating law, Q scales per bq rows, K
    and V per 64-row block), else the 16-bit one.  Returns the train_fwd dict
    (o, o_s, o_l, lse, den, qphi, htot, ztot, Hall, comp, lut_aug).
    """
    _need_gpu(q, k, v, lut)
    q, k, v = (_bhld(t, "qkv") for t in (q, k, v))
    B, H, L, D = q.shape
    nb, mq = -(-L // E_TILE), -(-L // bq)
    lut = lut.to(torch.int32).contiguous()
    if lut.dim() != 4 or tuple(lut.shape[:3]) != (B, H, mq):
        raise ValueError(f"lut: expected (B, H, {mq}, T), got {tuple(lut.shape)}")
    st = linear_states_qat(k, v, with_vt=not int8)
    if int8:
        qz = quant_train(q, k, v)
        qz["q8"], qz["qs"] = quantize_trunc(q, bq)
        o_s, lse, qphi = sparse_fwd_int8(q, qz["q8"], qz["qs"], bq, qz["k8"], qz["ks"],
                                         qz["v8f"], qz["vs"], lut, bq)
    else:
        o_s, lse, qphi = sparse_fwd_16(q, k, st["vt"], lut, bq)
    comp = complement(st, lut, nb, check_ids=False)
    if lut.shape[-1] <= SCORE_FORM_MAX_J:
        o, o_l, den = linear_mix_score(qphi, k, v, st, lut, o_s, alpha, eps_l, bq=bq)
    else:
        o, o_l, den = linear_mix_qat(qphi, comp, st["Hall"], o_s, alpha, eps_l, bq=bq)
    return dict(o=o, o_s=o_s, o_l=o_l, lse=lse, den=den, qphi=qphi,
                htot=st["Hall"].to(q.dtype).float(), ztot=st["zall"], Hall=st["Hall"], comp=comp,
                lut_aug=lut)


# ---------------------------------------------------------------------------
# Inference forward of the 1-D SLA2 module (SLA2.forward without gradients,
# models/sla2_vendor/core.py:93-128): the INT8 sparse branch of
# sparse_attention_int8 (or the 16-bit one), the state-subtraction linear
# branch of complement_linear_states and the alpha mix.
# ---------------------------------------------------------------------------

def quantize_trunc(x, E=E_TILE):
    """x (B,H,L,D) 16-bit -> (xq int8, xs fp32 (B,H,ceil(L/E))), the truncating law."""
    _need_gpu(x)
    x = _bhld(x, "x")
    B, H, L, D = x.shape
    xq = torch.empty_like(x, dtype=torch.int8)
    xs = torch.empty(B, H, -(-L // E), device=x.device, dtype=torch.float32)
    _lib.check(_lib.load().sla2h_quantize_trunc(x.data_ptr(), _dtype_code(x), B * H, L, D, E,
                                                xq.data_ptr(), xs.data_ptr(), _stream(x.device)),
               "sla2h_quantize_trunc")
    return xq, xs


def quantize_v8f(v, E=E_TILE):
    """V (B,H,L,64) 16-bit -> (v8f int8 (B,H,Nb,4096) fragment order, vs fp32 (B,H,Nb))."""
    _need_gpu(v)
    v = _bhld(v, "v")
    B, H, L, D = v.shape
    nb = -(-L // E)
    v8f = torch.empty(B, H, nb, 4096, device=v.device, dtype=torch.int8)
    vs = torch.empty(B, H, nb, device=v.device, dtype=torch.float32)
    _lib.check(_lib.load().sla2h_quantize_v8f(v.data_ptr(), _dtype_code(v), B * H, L, D, E,
                                              v8f.data_ptr(), vs.data_ptr(), _stream(v.device)),
               "sla2h_quantize_v8f")
    return v8f, vs


def sparse_fwd_int8(q, q8, qs, qblock, k8, ks, v8f, vs, lut, bq, scale=None, phi_out=True):
    """Inference INT8 sparse branch -> (o_s 16-bit, lse fp32, qphi 16-bit | None)."""
    _need_gpu(q, q8, k8, v8f, lut)
    B, H, L, D = q.shape
    lut = lut.to(torch.int32).contiguous()
    mq = -(-L // bq)
    if lut.dim() != 4 or tuple(lut.shape[:3]) != (B, H, mq):
        raise ValueError(f"lut: expected (B, H, {mq}, T), got {tuple(lut.shape)}")
    scale = D ** -0.5 if scale is None else scale
    o_s = torch.empty_like(q)
    lse = torch.empty(B, H, L, device=q.device, dtype=torch.float32)
    qphi = torch.empty_like(q) if phi_out else None
    _lib.check(_lib.load().sla2h_sparse_fwd_int8(
        q.data_ptr(), q8.data_ptr(), qs.data_ptr(), qblock, k8.data_ptr(), ks.data_ptr(),
        v8f.data_ptr(), vs.data_ptr(), lut.data_ptr(), _dtype_code(q), B, H, L, D, bq,
        lut.shape[-1], float(scale), o_s.data_ptr(), lse.data_ptr(), _ptr(qphi),
        _stream(q.device)), "sla2h_sparse_fwd_int8")
    return o_s, lse, qphi


def hblocks_states(k, v, with_sums=False, with_vt=False):
    """Inference states of every key block -> dict(Hb, zb [, Hall, zall] [, vt])."""
    _need_gpu(k, v)
    k, v = _bhld(k, "k"), _bhld(v, "v")
    B, H, L, D = k.shape
    nb = -(-L // E_TILE)
    f32, dev = torch.float32, k.device
    st = {"Hb": torch.empty(B, H, nb, D, D, device=dev, dtype=f32),
          "zb": torch.empty(B, H, nb, D, device=dev, dtype=f32)}
    if with_sums:
        st["Hall"] = torch.empty(B, H, D, D, device=dev, dtype=f32)
        st["zall"] = torch.empty(B, H, D, device=dev, dtype=f32)
    if with_vt:
        st["vt"] = torch.empty(B, H, nb, D, E_TILE, device=dev, dtype=v.dtype)
    _lib.check(_lib.load().sla2h_hblocks_states(
        k.data_ptr(), v.data_ptr(), _dtype_code(k), B, H, L, D, E_TILE, st["Hb"].data_ptr(),
        st["zb"].data_ptr(), _ptr(st.get("Hall")), _ptr(st.get("zall")), _ptr(st.get("vt")),
        _stream(dev)), "sla2h_hblocks_states")
    return st


def lin_fwd3(qphi, comp, o_s, alpha, bq, eps_l=1e-5):
    """Linear branch + mix of the inference path -> o (16-bit)."""
    _need_gpu(qphi, comp, o_s)
    B, H, L, D = qphi.shape
    a = _alpha_rows(alpha, H, -(-L // bq), qphi.device)
    o = torch.empty_like(o_s)
    _lib.check(_lib.load().sla2h_lin_fwd3(
        qphi.data_ptr(), comp.data_ptr(), o_s.data_ptr(), a.data_ptr(), a.stride(0),
        _dtype_code(qphi), B, H, L, D, bq, float(eps_l), o.data_ptr(), _stream(qphi.device)),
        "sla2h_lin_fwd3")
    return o


def sla2_infer(q, k, v, alpha, lut, bq, use_int8=True, qblock=None, eps_l=1e-5,
               return_parts=False):
    """SLA2 inference forward on given routing.

    q, k, v: (B,H,L,64) 16-bit, natural order; alpha (H, ceil(L/bq)) after the
    sigmoid; lut (B,H,ceil(L/bq),T) routed 64-row key blocks.  use_int8: the
    INT8 sparse branch with Q scales per qblock rows (default bq), else the
    16-bit one.  Returns o (16-bit) [, dict of the intermediates].
    """
    _need_gpu(q, k, v, lut)
    q, k, v = (_bhld(t, "qkv") for t in (q, k, v))
    B, H, L, D = q.shape
    nb = -(-L // E_TILE)
    lut = lut.to(torch.int32).contiguous()
    st = hblocks_states(k, v, with_vt=not use_int8)
    if use_int8:
        qb = bq if qblock is None else qblock
        q8, qs = quantize(q, qb)
        k8, ks = quantize(k)
        v8f, vs = quantize_v8f(v)
        o_s, lse, qphi = sparse_fwd_int8(q, q8, qs, qb, k8, ks, v8f, vs, lut, bq)
    else:
        o_s, lse, qphi = sparse_fwd_16(q, k, st["vt"], lut, bq)
    comp = complement(st, lut, nb, check_ids=False)
    o = lin_fwd3(qphi, comp, o_s, alpha, bq, eps_l)
    if return_parts:
        return o, dict(o_s=o_s, lse=lse, qphi=qphi, comp=comp, **st)
    return o


def sla2_infer_fused(q, k, v, alpha, lut, bq, use_int8=True, block_m=None, eps_l=1e-5,
                     scale=None):
    """SLA2 inference forward with the fused Algorithm-2 kernel's arithmetic
    (sla2_forward_fused, models/sla2_vendor/kernel_fused.py:127-160): Q scales
    per block_m rows (default max(32, bq // 2), as SLA2.forward picks), o_s in
    fp32 into the mix, the score-form linear branch against the whole-sequence
    state.  alpha (H, ceil(L/bq)) or a head-shared (ceil(L/bq),) row.
    Returns o (16-bit)."""
    _need_gpu(q, k, v, lut)
    q, k, v = (_bhld(t, "qkv") for t in (q, k, v))
    B, H, L, D = q.shape
    mq = -(-L // bq)
    lut = lut.to(torch.int32).contiguous()
    if lut.dim() != 4 or tuple(lut.shape[:3]) != (B, H, mq):
        raise ValueError(f"lut: expected (B, H, {mq}, T), got {tuple(lut.shape)}")
    block_m = block_m or max(32, bq // 2)
    alpha = torch.as_tensor(alpha).detach().to(q.device, torch.float32)
    if alpha.dim() == 1:
        alpha, stride = alpha.contiguous(), 0
    else:
        alpha = _alpha_rows(alpha, H, mq, q.device)
        stride = alpha.stride(0)
    if alpha.shape[-1] != mq:
        raise ValueError(f"alpha: expected {mq} query blocks, got {alpha.shape[-1]}")
    st = linear_states_qat(k, v, with_vt=not use_int8)
    q8 = qs = k8 = ks = v8f = vs = None
    if use_int8:
        q8, qs = quantize(q, block_m)
        k8, ks = quantize(k)
        v8f, vs = quantize_v8f(v)
    lib = _lib.load()
    ws = torch.empty(lib.sla2h_sla2_fused_workspace_bytes(B, H, L, D), device=q.device,
                     dtype=torch.uint8)
    o = torch.empty_like(q)
    scale = D ** -0.5 if scale is None else scale
    _lib.check(lib.sla2h_sla2_forward_fused(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(q8), _ptr(qs), block_m, _ptr(k8),
        _ptr(ks), _ptr(v8f), _ptr(vs), _ptr(st.get("vt")), st["Hall"].data_ptr(),
        st["zall"].data_ptr(), lut.data_ptr(), lut.shape[-1], alpha.data_ptr(), stride,
        _dtype_code(q), B, H, L, D, bq, float(scale), float(eps_l), ws.data_ptr(),
        o.data_ptr(), _stream(q.device)), "sla2h_sla2_forward_fused")
    return o


# ---------------------------------------------------------------------------
# DiT block, training forward / backward: fused SituAndMul
# (models/imf_dit_video.py:136-171)
# ---------------------------------------------------------------------------
_SITU_DTYPES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _rows_view(t):
    """(..., F) with a unit last stride -> (rows, F, row stride), without a copy
    when the leading dimensions collapse to one strided dimension."""
    F = t.shape[-1]
    v = t.reshape(-1, F)
    if v.stride(-1) != 1 or (v.shape[0] > 1 and v.stride(0) < F):
        v = v.contiguous()
    return v, F, max(v.stride(0), F)


def situ_mul_fwd(gate, up, beta, linear_beta=None):
    """h = beta tanh(gate / beta) sigmoid(gate) * u' (u' = lb tanh(up / lb) with
    a soft clamp, else up), fp32 arithmetic, in gate's dtype, shape of gate."""
    _need_gpu(gate, up)
    if gate.shape != up.shape or gate.dtype != up.dtype or gate.dtype not in _SITU_DTYPES:
        raise ValueError("gate and up must share shape and a 16-bit or fp32 dtype")
    g2, F, sg = _rows_view(gate)
    u2, _, su = _rows_view(up)
    out = torch.empty(gate.shape, device=gate.device, dtype=gate.dtype)
    _lib.check(_lib.load().sla2h_situ_mul_fwd(
        g2.data_ptr(), u2.data_ptr(), _SITU_DTYPES[gate.dtype], g2.shape[0], F, sg, su,
        float(beta), float(linear_beta or 0.0), out.data_ptr(), _stream(gate.device)),
        "sla2h_situ_mul_fwd")
    return out


def situ_mul_bwd(dh, gate, up, beta, linear_beta=None):
    """Gradients (dgate, dup) of situ_mul_fwd for the output gradient dh."""
    _need_gpu(dh, gate, up)
    g2, F, sg = _rows_view(gate)
    u2, _, su = _rows_view(up)
    dh = dh.to(gate.dtype).contiguous()
    dgate = torch.empty(gate.shape, device=gate.device, dtype=gate.dtype)
    dup = torch.empty_like(dgate)
    _lib.check(_lib.load().sla2h_situ_mul_bwd(
        dh.data_ptr(), g2.data_ptr(), u2.data_ptr(), _SITU_DTYPES[gate.dtype], g2.shape[0], F,
        sg, su, float(beta), float(linear_beta or 0.0), dgate.data_ptr(), dup.data_ptr(),
        _stream(gate.device)), "sla2h_situ_mul_bwd")
    return dgate, dup


# ---------------------------------------------------------------------------
# DiT block, training forward / backward: fused RMSNorm
# (models/imf_dit_video.py:121-133)
# ---------------------------------------------------------------------------
def rmsnorm_fwd(x, w, eps):
    """y = (x r).to(x.dtype) * w in fp32, r = rsqrt(mean(x^2) + eps); shape of x."""
    _need_gpu(x, w)
    if x.dtype not in _SITU_DTYPES:
        raise ValueError(f"RMSNorm input dtype {x.dtype} not supported")
    x2, D, sx = _rows_view(x)
    w = w.detach().to(torch.float32).contiguous()
    y = torch.empty(x.shape, device=x.device, dtype=torch.float32)
    _lib.check(_lib.load().sla2h_rmsnorm_fwd(
        x2.data_ptr(), _SITU_DTYPES[x.dtype], x2.shape[0], D, sx, w.data_ptr(), float(eps),
        y.data_ptr(), _stream(x.device)), "sla2h_rmsnorm_fwd")
    return y


def rmsnorm_bwd(dy, x, w, eps):
    """(dx in x's dtype, dw fp32) of rmsnorm_fwd for the output gradient dy."""
    _need_gpu(dy, x, w)
    x2, D, sx = _rows_view(x)
    w = w.detach().to(torch.float32).contiguous()
    dy = dy.to(torch.float32).contiguous()
    dx = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    dw = torch.empty(D, device=x.device, dtype=torch.float32)
    lib = _lib.load()
    ws = torch.empty(lib.sla2h_rmsnorm_bwd_workspace_bytes(x2.shape[0], D) // 4,
                     device=x.device, dtype=torch.float32)
    _lib.check(lib.sla2h_rmsnorm_bwd(
        x2.data_ptr(), _SITU_DTYPES[x.dtype], x2.shape[0], D, sx, w.data_ptr(), dy.data_ptr(),
        float(eps), dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), _stream(x.device)),
        "sla2h_rmsnorm_bwd")
    return dx, dw


_F16_CODES = {torch.float16: 0, torch.bfloat16: 1}


def gate_mul_fwd(a, g):
    """a * sigmoid(g) for 16-bit a, g of one shape and dtype (torch's rounding)."""
    _need_gpu(a, g)
    a, g = a.contiguous(), g.contiguous()
    out = torch.empty_like(a)
    _lib.check(_lib.load().sla2h_gate_mul_fwd(a.data_ptr(), g.data_ptr(), _F16_CODES[a.dtype],
                                              a.numel(), out.data_ptr(), _stream(a.device)),
               "sla2h_gate_mul_fwd")
    return out


def gate_mul_bwd(dout, a, g):
    """(da, dg) of gate_mul_fwd for the output gradient dout."""
    _need_gpu(dout, a, g)
    dout, a, g = dout.to(a.dtype).contiguous(), a.contiguous(), g.contiguous()
    da, dg = torch.empty_like(a), torch.empty_like(g)
    _lib.check(_lib.load().sla2h_gate_mul_bwd(dout.data_ptr(), a.data_ptr(), g.data_ptr(),
                                              _F16_CODES[a.dtype], a.numel(), da.data_ptr(),
                                              dg.data_ptr(), _stream(a.device)),
               "sla2h_gate_mul_bwd")
    return da, dg


def _half_args(t):
    """(tensor, dtype code, sb, st, sh) of a (B, L, H, 32) half (H may be 1 and
    broadcast: head stride 0)."""
    sb, st, sh, sc = t.stride()
    if sc != 1:
        raise ValueError("attention operand halves need unit channel stride")
    return t, _SITU_DTYPES[t.dtype], sb, st, (0 if t.shape[2] == 1 else sh)


def attn_in_fwd(halves, H):
    """(B, H, L, 64) fp16 operand from two (B, L, H|1, 32) halves (lo: channels
    0..31, hi: 32..63; fp32 or 16-bit lo, 16-bit hi) -- the sublayer's
    torch.cat(...).permute(0, 2, 1, 3).half() in one pass."""
    lo, hi = halves
    _need_gpu(lo, hi)
    B, L = lo.shape[:2]
    out = torch.empty(B, H, L, 64, device=lo.device, dtype=torch.float16)
    a, b = _half_args(lo), _half_args(hi)
    _lib.check(_lib.load().sla2h_attn_in_fwd(
        a[0].data_ptr(), *a[1:], b[0].data_ptr(), *b[1:], B, H, L, out.data_ptr(),
        _stream(lo.device)), "sla2h_attn_in_fwd")
    return out


def attn_in_bwd(dout, dlo, dhi):
    """Gradients of the two halves of attn_in_fwd from the (B, H, L, 64) fp16
    gradient, written into dlo and dhi (preallocated (B, L, H|1, 32) tensors
    or views in the halves' dtypes; a head-shared dhi gets the sum over the
    heads)."""
    _need_gpu(dout, dlo, dhi)
    B, H, L, _ = dout.shape
    dout = dout.to(torch.float16).contiguous()
    a, b = _half_args(dlo), _half_args(dhi)
    _lib.check(_lib.load().sla2h_attn_in_bwd(
        dout.data_ptr(), a[0].data_ptr(), *a[1:], b[0].data_ptr(), *b[1:], B, H, L,
        _stream(dout.device)), "sla2h_attn_in_bwd")


def attn_gate_fwd(o, g):
    """round16(fp32(o) sigmoid16(g)) as (B, L, H * 64) in g's dtype, from the
    op's (B, H, L, 64) fp16 output o and the gate logits g (B, L, H * 64)."""
    _need_gpu(o, g)
    B, H, L, D = o.shape
    o, g = o.contiguous(), g.contiguous()
    out = torch.empty(B, L, H * D, device=o.device, dtype=g.dtype)
    _lib.check(_lib.load().sla2h_attn_gate_fwd(o.data_ptr(), g.data_ptr(), _F16_CODES[g.dtype],
                                               B, H, L, out.data_ptr(), _stream(o.device)),
               "sla2h_attn_gate_fwd")
    return out


def attn_gate_bwd(dy, o, g):
    """(do (B, H, L, 64) fp16, dg) of attn_gate_fwd for the output gradient dy."""
    _need_gpu(dy, o, g)
    B, H, L, D = o.shape
    dy, o, g = dy.to(g.dtype).contiguous(), o.contiguous(), g.contiguous()
    do, dg = torch.empty_like(o), torch.empty_like(g)
    _lib.check(_lib.load().sla2h_attn_gate_bwd(dy.data_ptr(), o.data_ptr(), g.data_ptr(),
                                               _F16_CODES[g.dtype], B, H, L, do.data_ptr(),
                                               dg.data_ptr(), _stream(o.device)),
               "sla2h_attn_gate_bwd")
    return do, dg


def rmsnorm_fwd16(x, w, eps, dtype):
    """round16(rmsnorm_fwd(x, w, eps)) in `dtype` (bf16 / fp16) for an fp32 x of
    a power-of-two width <= 512: the norm and the autocast cast of its output
    in one pass."""
    _need_gpu(x, w)
    if x.dtype != torch.float32 or dtype not in _F16_CODES:
        raise ValueError("rmsnorm_fwd16: fp32 x and a 16-bit output dtype")
    x2, D, sx = _rows_view(x)
    w = w.detach().to(torch.float32).contiguous()
    y = torch.empty(x.shape, device=x.device, dtype=dtype)
    _lib.check(_lib.load().sla2h_rmsnorm_fwd16(
        x2.data_ptr(), x2.shape[0], D, sx, w.data_ptr(), float(eps), _F16_CODES[dtype],
        y.data_ptr(), _stream(x.device)), "sla2h_rmsnorm_fwd16")
    return y


def rmsnorm_bwd_sum(dys, x, w, eps, dadd=None):
    """(dx fp32, dw fp32) of rmsnorm_fwd16 for output gradients `dys` (1 to 3
    tensors of one 16-bit dtype, summed in fp32 in list order); dadd (fp32 or
    None) is added to dx."""
    _need_gpu(x, w, *dys)
    if not 1 <= len(dys) <= 3 or len({d.dtype for d in dys}) != 1 or dys[0].dtype not in _F16_CODES:
        raise ValueError("rmsnorm_bwd_sum: 1 to 3 output gradients of one 16-bit dtype")
    x2, D, sx = _rows_view(x)
    w = w.detach().to(torch.float32).contiguous()
    dys = [d.contiguous() for d in dys]
    dadd = None if dadd is None else dadd.to(torch.float32).contiguous()
    dx = torch.empty(x.shape, device=x.device, dtype=torch.float32)
    dw = torch.empty(D, device=x.device, dtype=torch.float32)
    lib = _lib.load()
    ws = torch.empty(lib.sla2h_rmsnorm_bwd_workspace_bytes(x2.shape[0], D) // 4,
                     device=x.device, dtype=torch.float32)
    ptr = lambda i: dys[i].data_ptr() if i < len(dys) else None
    _lib.check(lib.sla2h_rmsnorm_bwd_sum(
        x2.data_ptr(), x2.shape[0], D, sx, w.data_ptr(), ptr(0), ptr(1), ptr(2),
        _F16_CODES[dys[0].dtype], _ptr(dadd), float(eps), dx.data_ptr(), dw.data_ptr(),
        ws.data_ptr(), _stream(x.device)), "sla2h_rmsnorm_bwd_sum")
    return dx, dw


# ---------------------------------------------------------------------------
# DiT block, training forward / backward: RoPE (models/imf_dit_video.py:266-284)
# ---------------------------------------------------------------------------
def rope(x, cos_t, sin_t, inverse=False):
    """Pairs (2i, 2i+1) of x (b, l, H, hd) rotated by the angles of each token
    (by the negated angles with inverse); fp32 arithmetic, contiguous, x's dtype."""
    _need_gpu(x, cos_t, sin_t)
    if x.dim() != 4 or x.dtype not in _SITU_DTYPES or x.shape[-1] % 2:
        raise ValueError(f"rope: expected (b, l, H, even hd) float input, got {tuple(x.shape)}")
    if x.stride(-1) != 1:
        x = x.contiguous()
    B, L, H, hd = x.shape
    cos_t = cos_t.to(torch.float32).contiguous()
    sin_t = sin_t.to(torch.float32).contiguous()
    if tuple(cos_t.shape) != (L, hd // 2) or tuple(sin_t.shape) != (L, hd // 2):
        raise ValueError("rope: tables must be (l, hd // 2)")
    out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    _lib.check(_lib.load().sla2h_rope(
        x.data_ptr(), _SITU_DTYPES[x.dtype], B, L, H, hd, x.stride(0), x.stride(1), x.stride(2),
        cos_t.data_ptr(), sin_t.data_ptr(), int(bool(inverse)), out.data_ptr(),
        _stream(x.device)), "sla2h_rope")
    return out


# ---------------------------------------------------------------------------
# DiT block, training forward / backward: ReZero residual
# (models/imf_dit_video.py:529-532)
# ---------------------------------------------------------------------------
def residual_scale_fwd(x, a, s):
    """y = x + a * s (fp32; product and sum rounded separately)."""
    _need_gpu(x, a, s)
    x = x.contiguous()
    a = a.contiguous()
    D = x.shape[-1]
    s = s.detach().to(torch.float32).contiguous()
    y = torch.empty_like(x)
    _lib.check(_lib.load().sla2h_residual_scale_fwd(
        x.data_ptr(), a.data_ptr(), _SITU_DTYPES[a.dtype], s.data_ptr(), x.numel() // D, D,
        y.data_ptr(), _stream(x.device)), "sla2h_residual_scale_fwd")
    return y


def residual_scale_bwd(dy, a, s):
    """(da in a's dtype, ds fp32) of residual_scale_fwd; dx is dy itself."""
    _need_gpu(dy, a, s)
    dy = dy.to(torch.float32).contiguous()
    a = a.contiguous()
    D = a.shape[-1]
    rows = a.numel() // D
    s = s.detach().to(torch.float32).contiguous()
    da = torch.empty_like(a)
    ds = torch.empty(D, device=a.device, dtype=torch.float32)
    lib = _lib.load()
    ws = torch.empty(lib.sla2h_residual_scale_bwd_workspace_bytes(rows, D) // 4,
                     device=a.device, dtype=torch.float32)
    _lib.check(lib.sla2h_residual_scale_bwd(
        dy.data_ptr(), a.data_ptr(), _SITU_DTYPES[a.dtype], s.data_ptr(), rows, D,
        da.data_ptr(), ds.data_ptr(), ws.data_ptr(), _stream(a.device)),
        "sla2h_residual_scale_bwd")
    return da, ds
