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
    """Pick, for every bq-row query block, the T = max(1, int(topk_frac * Nb))
    key blocks (bk = 64 rows) whose pooled means score highest against the
    query block's pooled mean (after the optional (D, D) projections).

    q, k are (B, H, L, D); returns the block ids as a (B, H, ceil(L/bq), T)
    int32 tensor, best first, and T.  The hard selection is computed in one
    pinned fp32 order on the GPU (ties go to the lower block id).  The
    reference centres the pooled keys first (smooth-k); that moves each row of
    scores by one constant and cannot change which blocks win.
    """
    dt = _c16(q).dtype
    qc, kc = _c16(q).to(dt), _c16(k).to(dt)
    return ops.route_1d(qc, kc, topk_frac, bq, bk, proj_q, proj_k)


@torch.no_grad()
def sla2_mla_jvp(q, k, v, dq, dk, dv, alpha, topk_frac, bq, bk, lut=None, T=None, block_m=64):
    """The 1-D SLA2 attention of (q, k, v) and its directional derivative along
    (dq, dk, dv), in one pass.

    Every query block of bq rows attends exactly (softmax with scale D^-1/2)
    to its routed key blocks of bk = 64 rows and, through the softmax feature
    map, linearly to all the others; alpha (H, ceil(L/bq)) after the sigmoid,
    or a scalar, mixes the two per query block.  lut / T skip the router (for
    example to reuse the routing of the primal pass); without them the router
    of route_blocks picks topk_frac of the key blocks.  All six tensors are
    (B, H, L, 64); block_m is accepted for the reference's signature (it must
    divide bq; the kernel's work unit is fixed).  Returns (o, do), (B, H, L, 64)
    fp32.
    """
    return _sla2_mla_jvp(q, k, v, dq, dk, dv, alpha, topk_frac, bq, bk, lut, T, block_m, True)


def _sla2_mla_jvp(q, k, v, dq, dk, dv, alpha, topk_frac, bq, bk, lut, T, block_m, check_ids):
    """sla2_mla_jvp; check_ids=False skips the range check of a LUT that comes
    straight from route_blocks (the check reduces the LUT and reads the result
    back to the host, a synchronisation per call)."""
    B, H, L, D = q.shape
    if bq % block_m != 0:
        raise ValueError(f"block_m must divide bq: {block_m}, {bq}")
    dt = _c16(q).dtype
    qc, kc, vc, dqc, dkc, dvc = (t.to(dt).contiguous() for t in (q, k, v, dq, dk, dv))
    if lut is None:
        lut, T = ops.route_1d(qc, kc, topk_frac, bq, bk)
    else:
        lut = lut.to(device=q.device, dtype=torch.int32).contiguous()
        if check_ids:
            ops.check_lut_ids(lut, -(-L // bk))
    mq = -(-L // bq)
    if torch.is_tensor(alpha) and alpha.dim() == 2:
        a = alpha.detach().to(q.device, torch.float32)
    else:
        a = torch.full((H, mq), float(alpha), device=q.device, dtype=torch.float32)
    return ops.jvp_1d(qc, kc, vc, dqc, dkc, dvc, a, lut.to(q.device), bq)


def sla2_dense_ref(q, k, v, lut, alpha, bq, bk):
    """Dense O(L^2) form of sla2_mla_jvp's primal, for tests (differentiable;
    torch on the inputs' device).  Token (i, j) takes the exact branch when
    key block j // bk is in the LUT row of query block i // bq, the linear
    branch otherwise; alpha (H, ceil(L/bq)) mixes the two per query block.
    q, k, v (B, H, L, D) fp32, lut (B, H, ceil(L/bq), T) -> (B, H, L, D).
    """
    B, H, L, D = q.shape
    qblk = torch.arange(L, device=q.device) // bq
    kblk = torch.arange(L, device=q.device) // bk
    routed = torch.zeros(B, H, lut.shape[2], -(-L // bk), device=q.device)
    routed.scatter_(-1, lut.long(), 1.0)
    exact = routed[:, :, qblk][..., kblk] > 0                   # (B, H, L, L)
    scores = (q @ k.transpose(-1, -2)) * D ** -0.5
    o_s = torch.softmax(scores.masked_fill(~exact, float("-inf")), dim=-1) @ v
    kernel = F.softmax(q, dim=-1) @ F.softmax(k, dim=-1).transpose(-1, -2)
    kernel = kernel.masked_fill(exact, 0.0)
    o_l = (kernel @ v) / (kernel.sum(-1, keepdim=True) + _EPS_L)
    a = alpha[:, qblk].reshape(1, H, L, 1)
    return a * o_s + (1.0 - a) * o_l
