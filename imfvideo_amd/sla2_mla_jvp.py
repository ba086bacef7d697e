"""1-D SLA2 sparse-linear attention and its forward-mode JVP (the MLA variant).

Same names, signatures and return conventions as the reference's
models/sla2_mla_jvp.py, computed by gfx950 HIP kernels through the C ABI of
include/sla2h.h:

  route_blocks   (reference :75-100)  block means (bq-row query blocks, 64-row key
                                      blocks) + optional projections, pooled scores,
                                      top-k -- sla2h_pool_blocks, sla2h_route_topk
  sla2_mla_jvp   (reference :348-385) states + complement GEMM + the fused JVP
                                      kernel with 16-bit scores -- sla2h_fwd_jvp_1d
  sla2_dense_ref (reference :388-418) the reference's dense fp32 test utility

Inputs are (B, H, L, D) in natural token order, D = 64, key blocks of 64 rows
(bk = 64), query blocks of bq = 64, 128 or 256 rows.  16-bit inputs keep their
type; fp32 inputs are rounded to fp16 (the reference's MMA path).
"""

import torch
import torch.nn.functional as F

from . import ops

__all__ = ["route_blocks", "sla2_mla_jvp", "sla2_dense_ref"]

_EPS_L = 1e-5


def _c16(x):
    return (x if x.dtype in (torch.float16, torch.bfloat16) else x.to(torch.float16)).contiguous()


@torch.no_grad()
def route_blocks(q, k, topk_frac, bq, bk, proj_q=None, proj_k=None):
    """SLA2 router: pooled-score hard top-k over key blocks.

    Args:
        q, k: (B, H, L, D) primal queries / keys.
        topk_frac: fraction of key blocks routed to the sparse branch.
        bq, bk: query / key block lengths (bk = 64).
        proj_q, proj_k: optional (D, D) router projection weights.

    Returns:
        lut: (B, H, ceil(L/bq), T) int32 routed key-block ids (descending score).
        T: topk count (int).

    The reference subtracts the mean pooled key before scoring (smooth-k); that
    adds a per-row constant to the scores and leaves the selection unchanged.
    """
    dt = _c16(q).dtype
    qc, kc = _c16(q).to(dt), _c16(k).to(dt)
    return ops.route_1d(qc, kc, topk_frac, bq, bk, proj_q, proj_k)


@torch.no_grad()
def sla2_mla_jvp(q, k, v, dq, dk, dv, alpha, topk_frac, bq, bk, lut=None, T=None, block_m=64):
    """SLA2 attention (primal, tangent) from qkv dual pairs.

    Args:
        q, k, v: (B, H, L, D) primal (D == Dv == 64).
        dq, dk, dv: (B, H, L, D) tangents.
        alpha: (H, Mb) mixing ratio in (0,1) (already sigmoided), or scalar.
        topk_frac: routed fraction of key blocks (ignored when lut given).
        bq, bk: query / key block lengths.
        lut, T: optional precomputed routing (from the primal training pass).
        block_m: accepted for the reference's signature; the kernel's work unit
            is fixed at 32 query rows.

    Returns:
        (o, do): (B, H, L, D) fp32 SLA2 output and tangent.
    """
    B, H, L, D = q.shape
    if bq % block_m != 0:
        raise ValueError(f"block_m must divide bq: {block_m}, {bq}")
    dt = _c16(q).dtype
    qc, kc, vc, dqc, dkc, dvc = (t.to(dt).contiguous() for t in (q, k, v, dq, dk, dv))
    if lut is None:
        lut, T = ops.route_1d(qc, kc, topk_frac, bq, bk)
    mq = -(-L // bq)
    if torch.is_tensor(alpha) and alpha.dim() == 2:
        a = alpha.detach().to(q.device, torch.float32)
    else:
        a = torch.full((H, mq), float(alpha), device=q.device, dtype=torch.float32)
    return ops.jvp_1d(qc, kc, vc, dqc, dkc, dvc, a, lut.to(q.device), bq)


def sla2_dense_ref(q, k, v, lut, alpha, bq, bk):
    """Dense fp32 SLA2 reference (mask from LUT), differentiable, for tests.

    The reference's O(L^2) test utility, kept for API parity: plain torch on
    whatever device the inputs live on.
    """
    B, H, L, D = q.shape
    Nb = (L + bk - 1) // bk
    mc = torch.zeros(B, H, lut.shape[2], Nb, device=q.device)
    mc.scatter_(-1, lut.long(), 1.0)
    m = mc.repeat_interleave(bq, dim=-2).repeat_interleave(bk, dim=-1)[..., :L, :L]
    s = (q @ k.transpose(-1, -2)) * D ** -0.5
    p = torch.softmax(s.masked_fill(m <= 0, float("-inf")), dim=-1)
    o_s = p @ v
    w = (F.softmax(q, dim=-1) @ F.softmax(k, dim=-1).transpose(-1, -2)) * (1.0 - m)
    o_l = (w @ v) / (w.sum(-1, keepdim=True) + _EPS_L)
    a = alpha.repeat_interleave(bq, dim=-1)[:, :L].view(1, H, L, 1)
    return a * o_s + (1.0 - a) * o_l
