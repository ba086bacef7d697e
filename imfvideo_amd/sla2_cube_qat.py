"""SLA2 cube-tile sparse-linear attention with INT8 QAT: forward and forward-mode JVP.

Same module and function names, signatures and return conventions as the
reference's models/sla2_cube_qat.py, computed by gfx950 HIP kernels through
the C ABI of include/sla2h.h:

  sla2_cube_qat_jvp_fused  (reference :605-672)  quant+pool -> route -> states
                           -> complement -> fused attention kernel
  sla2_cube_qat_jvp        (reference :210-289)  same kernels
  _sparse_primal_only      (reference :172-207)  sparse branch only
  SLA2CubeQATAttentionImpl (reference :295-439)  the attn_impl module

Inputs are (B, H, L, D) tile-major tensors (L = Np*E + P, the P prefix
tokens last).  16-bit inputs keep their type (bf16 or fp16); fp32 inputs are
rounded to ``COMPUTE_DTYPE`` (bfloat16) -- the reference rounds to fp16.
"""

import math

import torch
import torch.nn as nn

from . import ops
from .mla_video_sparse_jvp import _plenty_of_vram, route_tiles, route_tiles_fast, tile_permutation

__all__ = ["SLA2CubeQATAttentionImpl", "sla2_cube_qat_jvp", "sla2_cube_qat_jvp_fused"]

_EPS_L = 1e-5
COMPUTE_DTYPE = torch.bfloat16


def _c16(x, dtype=None):
    if dtype is None:
        dtype = x.dtype if x.dtype in (torch.float16, torch.bfloat16) else COMPUTE_DTYPE
    return x.to(dtype).contiguous()


def _alpha_tensor(alpha, H, Mb, device):
    """(H, Mb) fp32 mix ratio from a tensor or a scalar."""
    if torch.is_tensor(alpha) and alpha.dim() == 2:
        return alpha.detach().to(device, torch.float32)
    a = float(alpha.item() if torch.is_tensor(alpha) else alpha)
    return torch.full((H, Mb), a, device=device, dtype=torch.float32)


def _check_geometry(L, Np, E, prefix_len):
    assert E == ops.E_TILE, f"E must be {ops.E_TILE} (quantisation block = tile), got {E}"
    assert L == Np * E + prefix_len, (L, Np, E, prefix_len)


@torch.no_grad()
def sla2_cube_qat_jvp_fused(q, k, v, dq, dk, dv, alpha, topk_frac, Np, E, prefix_len,
                            proj_q=None, proj_k=None, lut=None, T=None):
    """Fused cube-QAT JVP: both branches and the mix in one attention kernel.

    Args:
        q..dv: (B, H, L, D) primal / tangent, tile-major order.
        alpha: (H, Mb) mixing ratio in (0, 1) (after the sigmoid), or scalar.
        topk_frac: routed fraction of the Np video tiles (ignored when lut given).
        Np, E, prefix_len: tiling geometry; E = 64.
        proj_q, proj_k: optional (D, D) router projections.
        lut, T: optional precomputed routing (B, H, Mb, T).

    Returns:
        (o, do): (B, H, L, D) fp32.
    """
    B, H, L, D = q.shape
    _check_geometry(L, Np, E, prefix_len)
    dt = _c16(q).dtype
    qc, kc, vc, dqc, dkc, dvc = (_c16(t, dt) for t in (q, k, v, dq, dk, dv))
    Mb = -(-L // E)
    a = _alpha_tensor(alpha, H, Mb, q.device)
    return ops.cube_jvp(qc, kc, vc, dqc, dkc, dvc, a, topk_frac, Np, prefix_len,
                        proj_q, proj_k, lut=lut, T=T)


def sla2_cube_qat_jvp(q, k, v, dq, dk, dv, alpha, topk_frac, Np, E, prefix_len,
                      proj_q=None, proj_k=None, lut=None, T=None):
    """Cube-block QAT attention (primal, tangent) -- reference :210-289.

    Same kernels as ``sla2_cube_qat_jvp_fused``.  The reference's unfused
    variant differs from the fused one only at rounding level (fp16-accumulated
    tangent dots, unsigned linear-branch epsilon); this build serves both
    names with the fused kernel.
    """
    return sla2_cube_qat_jvp_fused(q, k, v, dq, dk, dv, alpha, topk_frac, Np, E, prefix_len,
                                   proj_q, proj_k, lut, T)


@torch.no_grad()
def _sparse_primal_only(q, k, v, lut, T, Np, E, prefix_len):
    """Primal sparse branch only (INT8 scores, 16-bit P.V) -> o_s (B,H,L,D) fp32."""
    B, H, L, D = q.shape
    _check_geometry(L, Np, E, prefix_len)
    dt = _c16(q).dtype
    qc, kc, vc = (_c16(t, dt) for t in (q, k, v))
    lut = lut.to(torch.int32).contiguous()
    q8, qs, k8, ks, _, _, kb = ops.quant_pool_qk(qc, kc, Np, E, with_kb=True)
    st = ops.linear_states(kc, vc, Np)
    o, _ = ops.fwd_jvp(qc, q8, k8, qs, ks, st, None, None, lut, Np, sparse_only=True, kb=kb)
    return o


class _CubeQATFunction(torch.autograd.Function):
    """Training op with the straight-through backward (reference :696-832).

    Same argument list as the reference.  ``use_int8`` picks the INT8 or the
    16-bit sparse branch of the forward; the backward is the same 16-bit
    recompute for both, as in the reference.  ``mask`` and ``a_index`` are
    accepted and unused: the kernels derive the per-tile selection from
    ``lut_aug`` on the device, and the alpha of a row is that of its 64-row
    block.
    """

    @staticmethod
    def forward(ctx, qh, kh, vh, alpha_logit, lut, lut_aug, mask, T, E, use_int8, a_index,
                n_tail=1, stats_out=None):
        assert E == ops.E_TILE, f"E must be {ops.E_TILE}, got {E}"
        B, H, L, D = qh.shape
        Np = -(-L // E) - n_tail
        a = torch.sigmoid(alpha_logit.detach().float())
        out = ops.train_fwd(qh, kh, vh, a, lut, Np, int8=bool(use_int8))
        if stats_out is not None:
            stats_out.copy_(out["lse"].amax(dim=(0, 2)))
        ctx.save_for_backward(qh, kh, vh, a, out["o_s"], out["o_l"], out["lse"], out["den"],
                              out["qphi"], out["Hall"], out["comp"], out["lut_aug"])
        return out["o"]

    @staticmethod
    def backward(ctx, do):
        qh, kh, vh, a, o_s, o_l, lse, den, qphi, Hall, comp, lut_aug = ctx.saved_tensors
        fwd = dict(o_s=o_s, o_l=o_l, lse=lse, den=den, qphi=qphi, Hall=Hall, comp=comp,
                   lut_aug=lut_aug)
        dq, dk, dv, d_alpha = ops.train_bwd(qh, kh, vh, a, fwd, do)
        return (dq, dk, dv, d_alpha, None, None, None, None, None, None, None, None, None)


class SLA2CubeQATAttentionImpl(nn.Module):
    """The cube-tile SLA2 attention as a DiT ``attn_impl`` (reference :295-439).

    Constructor arguments (the reference's, same names and defaults):
    ``head_dim`` is the per-head width of q, k and v (64); ``seq_len`` counts
    the prefix tokens plus the patch tokens of ``grid`` (frames, height,
    width); ``num_heads`` is H; ``tile`` is the 3-D tile whose volume E must
    be 64; ``topk`` is the fraction of the video tiles each query block routes
    to the exact branch; ``alpha_init`` sets every entry of ``alpha_logit``
    so that its sigmoid starts there; ``use_int8`` selects the INT8 sparse
    branch of the training forward (False: 16-bit scores and P.V);
    ``pre_permuted`` says the caller already keeps the tokens in tile order.

    forward(q, k, v) takes (b, l, H, hd) tensors, moves them to tile order in
    fp16 (as the reference does), routes on them without gradient (so
    proj_q / proj_k never receive one), and runs the training-forward kernels
    (``ops.train_fwd``: sparse branch, state-form linear branch, alpha mix),
    also under no_grad as the reference's guidance path does.  With gradients
    required the call goes through ``_CubeQATFunction`` (straight-through
    backward) and refreshes ``logit_max_log2`` (H,), the per-head maximum of
    the sparse branch's lse, for the QK-Clip step.
    """

    TILE_MAJOR = True

    def __init__(self, head_dim, seq_len, num_heads, grid, tile=(4, 4, 4), topk=0.03,
                 alpha_init=0.9, use_int8=True, pre_permuted=False):
        super().__init__()
        self.pre_permuted = pre_permuted
        self.E = tile[0] * tile[1] * tile[2]
        self.topk_frac = topk
        self.use_int8 = use_int8
        n_patch = grid[0] * grid[1] * grid[2]
        self.prefix_len = seq_len - n_patch
        perm, inv, self.Np = tile_permutation(grid, tile, self.prefix_len, torch.device("cpu"))
        self.register_buffer("perm", perm, persistent=False)
        self.register_buffer("inv", inv, persistent=False)
        self.n_tail = -(-self.prefix_len // self.E)
        self.Mb = self.Np + self.n_tail
        rows = torch.arange(seq_len)
        self.register_buffer("a_index", torch.clamp(rows // self.E, max=self.Mb - 1),
                             persistent=False)
        self.Nb = math.ceil(seq_len / self.E)
        self.proj_q = nn.Parameter(torch.eye(head_dim))
        self.proj_k = nn.Parameter(torch.eye(head_dim))
        init = torch.logit(torch.tensor(float(alpha_init)))
        self.alpha_logit = nn.Parameter(torch.full((num_heads, self.Mb), init.item()))

    def forward(self, q, k, v):
        """q, k, v: (b, l, H, hd) -> (b, l, H, hd) attention output in q.dtype."""

        def tm(x):
            x = x.permute(0, 2, 1, 3)
            if not self.pre_permuted:
                x = x[:, :, self.perm]
            return x.half().contiguous()

        o = self.forward_tile_major(tm(q), tm(k), tm(v))
        if self.pre_permuted:
            return o.permute(0, 2, 1, 3).to(q.dtype)
        return o[:, :, self.inv].permute(0, 2, 1, 3).to(q.dtype)

    def forward_tile_major(self, qh, kh, vh):
        """The op on operands already in its layout: qh, kh, vh (b, H, l, hd)
        fp16, tile-major rows, contiguous -> o (b, H, l, hd) fp16 in the same
        rows.  forward() is this between the reference's permute / .half() of
        q, k, v and the permute / cast back of o; a caller that keeps the
        sequence tile-major can build the operands and consume o directly."""
        B, H, L, D = qh.shape
        with torch.no_grad():
            lut, T = route_tiles_fast(qh, kh, self.topk_frac, self.Np, self.E, self.prefix_len,
                                      proj_q=self.proj_q, proj_k=self.proj_k)
        needs_grad = torch.is_grad_enabled() and (
            qh.requires_grad or kh.requires_grad or vh.requires_grad
            or self.alpha_logit.requires_grad)
        if needs_grad:
            if not hasattr(self, "logit_max_log2"):
                self.logit_max_log2 = torch.zeros(H, device=qh.device, dtype=torch.float32)
            lut_aug = ops.augment_lut(lut, self.Np, self.n_tail)
            return _CubeQATFunction.apply(qh, kh, vh, self.alpha_logit, lut, lut_aug, None, T,
                                          self.E, self.use_int8, self.a_index, self.n_tail,
                                          self.logit_max_log2)
        a = torch.sigmoid(self.alpha_logit.detach().float())
        return ops.train_fwd(qh, kh, vh, a, lut, self.Np, int8=self.use_int8)["o"]
