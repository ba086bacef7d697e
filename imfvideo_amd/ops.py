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


def quant_pool_qk(q, k, Np, E=E_TILE, proj_q=None, proj_k=None):
    """INT8 Q/K with per-block scales plus the router's pooled (projected) tiles.

    Returns q8, qs, k8, ks, qpool (B,H,Nb,D) fp32, kpool_t (B,H,D,Np) fp32.
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
    _lib.check(_lib.load().sla2h_quant_pool_qk(
        q.data_ptr(), k.data_ptr(), _dtype_code(q), B, H, L, D, E, Np,
        _ptr(pq), _ptr(pk), q8.data_ptr(), qs.data_ptr(), k8.data_ptr(), ks.data_ptr(),
        qpool.data_ptr(), kpool_t.data_ptr(), _stream(dev)), "sla2h_quant_pool_qk")
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


def complement(st, lut, Np):
    """Per-query-block complement records (uint8 (B,H,Mb,REC_BYTES))."""
    B, H, Mb, T = lut.shape
    lib = _lib.load()
    comp = torch.empty(B, H, Mb, REC_BYTES, device=lut.device, dtype=torch.uint8)
    ws = torch.empty(lib.sla2h_complement_workspace_bytes(B, H, Mb, Np), device=lut.device,
                     dtype=torch.uint8)
    g = lambda n: _ptr(st.get(n))
    _lib.check(lib.sla2h_complement(
        g("Hb"), g("dHb"), g("zb"), g("dzb"), lut.contiguous().data_ptr(), B, H, Mb, Np,
        E_TILE, T, ws.data_ptr(), comp.data_ptr(), _stream(lut.device)), "sla2h_complement")
    return comp


def fwd_jvp(q, q8, k8, qs, ks, st, comp, alpha, lut, Np, dq=None, scale=None, eps_l=1e-5,
            sparse_only=False):
    """The fused sparse+linear op (and JVP when dq is given) -> (o, do|None) fp32.

    The key side comes from k8/ks and the operand tiles of `st`
    (linear_states with tangents when dq is given).
    """
    _need_gpu(q, dq, alpha, lut)
    B, H, L, D = q.shape
    T = lut.shape[-1]
    tan = dq is not None
    if tan != ("dHb" in st):
        raise ValueError("fwd_jvp: the states must be built with tangents exactly when dq is given")
    scale = D ** -0.5 if scale is None else scale
    o = torch.empty(B, H, L, D, device=q.device, dtype=torch.float32)
    do = torch.empty_like(o) if tan else None
    if alpha is not None:
        alpha = alpha.detach().to(q.device, torch.float32)
        if alpha.dim() != 2 or alpha.stride(1) != 1:
            alpha = alpha.reshape(H, -1).contiguous()
    _lib.check(_lib.load().sla2h_fwd_jvp(
        q.data_ptr(), _ptr(dq), _ptr(st.get("kt")) if tan else None, st["vt"].data_ptr(),
        q8.data_ptr(), k8.data_ptr(), qs.data_ptr(),
        ks.data_ptr(), _ptr(comp), _ptr(alpha), 0 if alpha is None else alpha.stride(0),
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
    q8, qs, k8, ks, qpool, kpool_t = quant_pool_qk(q, k, Np, E, proj_q, proj_k)
    if lut is None:
        T = topk_count(topk_frac, Np)
        lut = route_topk(qpool, kpool_t, T, D ** -0.5)
    else:
        lut = lut.to(torch.int32).contiguous()
        T = lut.shape[-1]
    st = linear_states(k, v, Np, dk if tan else None, dv if tan else None, E, with_sums=False)
    comp = complement(st, lut, Np)
    o, do = fwd_jvp(q, q8, k8, qs, ks, st, comp, alpha, lut, Np, dq if tan else None)
    if return_aux:
        aux = dict(q8=q8, qs=qs, k8=k8, ks=ks, qpool=qpool, kpool_t=kpool_t, lut=lut, T=T,
                   comp=comp, **st)
        return o, do, aux
    return o, do
