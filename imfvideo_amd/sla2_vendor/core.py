"""SLA2: sparse-linear attention with a learnable router, on the gfx950 kernels
(reference: models/sla2_vendor/core.py).

    O   = a .* O_s + (1 - a) .* O_l,   a = sigmoid(alpha_logit) per (head, query block)
    O_s = softmax(Q K^T / sqrt(d) over the routed key blocks) V
    O_l = phi(Q) [phi(K)^T V over the other key blocks] / (phi(Q) . z + eps)

Query blocks of bq rows (64, 128 or 256), key blocks of bk = 64 rows.  With
gradients enabled the forward runs the training-forward kernels (16-bit
sparse branch, or with use_int8 the INT8 one of _attn_fwd_qat; 16-bit
state-form linear branch and mix) inside an autograd
Function whose backward is the straight-through HIP backward.  Without
gradients it runs the inference path (ops.sla2_infer): the INT8 sparse
branch of sparse_attention_int8 (or the 16-bit one), the state-subtraction
linear branch of complement_linear_states and the alpha mix.
"""

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import ops
from .router import Router


def softmax_feature_map(x):
    """The linear branch's feature map: a softmax across the D channels of every
    token of x (B, H, L, D), evaluated in fp32 and returned in x's dtype."""
    if x.dtype == torch.float32:
        return F.softmax(x, dim=-1)
    return F.softmax(x, dim=-1, dtype=torch.float32).to(x.dtype)


class _SLA2Function(torch.autograd.Function):
    """Training op of SLA2 (16-bit sparse + complement linear + alpha mix) with the
    straight-through backward.  Inputs (B,H,L,D) 16-bit contiguous."""

    @staticmethod
    def forward(ctx, qh, kh, vh, alpha_logit, lut, bq, use_int8):
        a = torch.sigmoid(alpha_logit.detach().float())
        out = ops.train_fwd_1d(qh, kh, vh, a, lut, bq, int8=use_int8)
        ctx.bq = bq
        ctx.save_for_backward(qh, kh, vh, a, out["o_s"], out["o_l"], out["lse"], out["den"],
                              out["qphi"], out["Hall"], out["comp"], out["lut_aug"])
        return out["o"]

    @staticmethod
    def backward(ctx, do):
        qh, kh, vh, a, o_s, o_l, lse, den, qphi, Hall, comp, lut_aug = ctx.saved_tensors
        fwd = dict(o_s=o_s, o_l=o_l, lse=lse, den=den, qphi=qphi, Hall=Hall, comp=comp,
                   lut_aug=lut_aug)
        dq, dk, dv, d_alpha = ops.train_bwd(qh, kh, vh, a, fwd, do, bq=ctx.bq)
        return dq, dk, dv, d_alpha, None, None, None


class SLA2(nn.Module):
    def __init__(self, head_dim, topk=0.03, bq=128, bk=64, tau=0.1, use_bf16=False, use_int8=True,
                 learnable_router=True, alpha_init=0.9, block_m=None, fused=False,
                 backend="cutedsl"):
        """Arguments keep the reference's names and defaults.  The head width
        must be 64 and key blocks 64 rows (bk); query blocks (bq) may be 64,
        128 or 256 rows.  topk is the share of key blocks each query block
        sends to the exact branch; tau the SoftTop-k temperature of the router;
        use_bf16 picks bf16 over fp16 as the 16-bit type; use_int8 quantises
        the exact branch; learnable_router gives the router trainable
        projections; alpha_init is the mixing weight every (head, query block)
        starts from.  fused selects the fused Algorithm-2 inference kernel
        (alpha averaged over heads, Q scales per block_m rows, by default
        max(32, bq // 2), o_s kept in fp32, the score-form linear branch).
        backend is accepted and ignored: one set of HIP kernels serves every
        backend name."""
        super().__init__()
        if bk != ops.E_TILE:
            raise ValueError(f"bk must be {ops.E_TILE}, got {bk}")
        if bq not in (64, 128, 256):
            raise ValueError(f"bq must be 64, 128 or 256, got {bq}")
        if block_m is not None and (block_m not in (32, 64, 128, 256) or bq % block_m):
            raise ValueError(f"block_m must divide bq and be 32..256, got {block_m}")
        self.dtype = torch.bfloat16 if use_bf16 else torch.float16
        self.topk, self.bq, self.bk = topk, bq, bk
        self.use_int8 = use_int8
        self.block_m, self.fused, self.backend = block_m, fused, backend
        self.router = Router(head_dim, bq=bq, bk=bk, tau=tau, learnable=learnable_router)
        self._alpha_init = alpha_init
        self.alpha_logit = None  # (H, Mb), created at the first forward unless set

    def _get_alpha(self, n_heads, n_qblocks, device):
        if self.alpha_logit is None or self.alpha_logit.shape != (n_heads, n_qblocks):
            init = torch.logit(torch.tensor(self._alpha_init))
            self.alpha_logit = nn.Parameter(
                torch.full((n_heads, n_qblocks), init.item(), device=device))
        return self.alpha_logit

    def forward(self, q, k, v, return_sparsity=False):
        """q, k, v: (B, H, L, D). Returns o: (B, H, L, D) in q.dtype."""
        out_dtype = q.dtype
        B, H, L, D = q.shape
        training = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad
                                                or v.requires_grad)
        qh, kh, vh = (t.to(self.dtype).contiguous() for t in (q, k, v))
        # the router scores the inputs in their own dtype (reference core.py:88)
        lut, topk = self.router.route(q, k, self.topk)
        alpha_logit = self._get_alpha(H, -(-L // self.bq), q.device)
        if training:
            o = _SLA2Function.apply(qh, kh, vh, alpha_logit, lut, self.bq, self.use_int8)
        else:
            # inference (core.py:98-128): INT8 or 16-bit sparse branch, the
            # state-subtraction linear branch and the mix
            a = torch.sigmoid(alpha_logit.detach().float())
            if self.fused:  # sla2_forward_fused: head-shared alpha, Q tiles of block_m
                o = ops.sla2_infer_fused(qh, kh, vh, a.mean(0), lut, self.bq,
                                         use_int8=self.use_int8, block_m=self.block_m)
            else:
                o = ops.sla2_infer(qh, kh, vh, a, lut, self.bq, use_int8=self.use_int8)
        if return_sparsity:
            return o.to(out_dtype), 1.0 - topk / -(-L // self.bk)
        return o.to(out_dtype)


# ---------------------------------------------------------------------------
# Dense references (plain torch, O(L^2)): the reference's correctness and
# stage-1 router utilities, kept for API parity.
# ---------------------------------------------------------------------------

def expand_mask(mc, bq, bk, L):
    """Spread a (B, H, Mb, Nb) block mask to its (B, H, L, L) token mask: token
    pair (i, j) takes the value of block pair (i // bq, j // bk)."""
    m = mc.repeat_interleave(bq, dim=-2).repeat_interleave(bk, dim=-1)
    return m[..., :L, :L]


def sla2_dense(q, k, v, mc, alpha, bq, bk):
    """SLA2 in dense fp32.  mc (B,H,Mb,Nb) hard int8 {0,1} or soft [0,1];
    alpha (Mb,) in (0,1)."""
    B, H, L, D = q.shape
    m = expand_mask(mc.float(), bq, bk, L)
    s = (q.float() @ k.float().transpose(-1, -2)) * D ** -0.5
    if mc.dtype == torch.int8:
        p = torch.softmax(s.masked_fill(m <= 0, float("-inf")), dim=-1)
    else:
        p = torch.softmax(s + torch.log(m + 1e-9), dim=-1)
    o_s = p @ v.float()
    qphi, kphi = softmax_feature_map(q), softmax_feature_map(k)
    w = (qphi.float() @ kphi.float().transpose(-1, -2)) * (1.0 - m)
    o_l = (w @ v.float()) / (w.sum(-1, keepdim=True) + 1e-5)
    a = alpha.repeat_interleave(bq)[:L].view(1, 1, L, 1)
    return a * o_s + (1.0 - a) * o_l


def full_attention(q, k, v):
    """Unmasked softmax attention with scale D^-1/2, computed in fp32:
    (B, H, L, D) inputs -> (B, H, L, D)."""
    D = q.shape[-1]
    s = (q.float() @ k.float().transpose(-1, -2)) * D ** -0.5
    return torch.softmax(s, dim=-1) @ v.float()
