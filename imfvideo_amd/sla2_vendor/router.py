"""Learnable SLA2 router (reference: models/sla2_vendor/router.py).

    Qbar = pool(Q) over bq-row blocks,  Kbar = pool(K) over bk-row blocks
    Pc   = proj_q(Qbar) proj_k(Kbar)^T * D^-0.5
    Mc   = top-k(k%, Pc) (hard) or SoftTop-k (stage-1 router training)

The hard selection runs on the HIP kernels (sla2h_pool_blocks +
sla2h_route_topk, canonical fp32 order, ties to the lower block).  The
reference's smooth-k (K minus its mean) shifts each score row by a constant
and so does not change the selection; the differentiable scores of
``scores`` / ``soft=True`` keep it.
"""

import torch
import torch.nn as nn

from .. import ops


def soft_topk(pc, k_frac, tau=0.1, n_iters=30):
    """SoftTop-k: sigmoid(pc/tau + lambda_row), lambda set by bisection so that
    each row sums to k_frac * (number of key blocks); lambda is detached.

    pc: (B, H, Mb, Nb) fp32 scores -> (B, H, Mb, Nb) soft mask in [0, 1].
    """
    x = pc.float() / tau
    target = k_frac * pc.shape[-1]
    lo = torch.full(pc.shape[:-1], -1e4, device=pc.device)
    hi = torch.full(pc.shape[:-1], 1e4, device=pc.device)
    with torch.no_grad():
        for _ in range(n_iters):
            mid = 0.5 * (lo + hi)
            over = torch.sigmoid(x + mid[..., None]).sum(-1) > target
            hi = torch.where(over, mid, hi)
            lo = torch.where(over, lo, mid)
    return torch.sigmoid(x + (0.5 * (lo + hi))[..., None])


class Router(nn.Module):
    """R(Q, K) -> block mask and LUT; proj_q / proj_k are identity-initialised
    nn.Linear(D, D, bias=False) in fp32 (state-dict names as the reference)."""

    def __init__(self, head_dim, bq=128, bk=64, tau=0.1, learnable=True):
        super().__init__()
        self.bq, self.bk, self.tau = bq, bk, tau
        self.learnable = learnable
        self.proj_q = nn.Linear(head_dim, head_dim, bias=False, dtype=torch.float32)
        self.proj_k = nn.Linear(head_dim, head_dim, bias=False, dtype=torch.float32)
        with torch.no_grad():
            self.proj_q.weight.copy_(torch.eye(head_dim))
            self.proj_k.weight.copy_(torch.eye(head_dim))
        if not learnable:
            for p in self.parameters():
                p.requires_grad_(False)

    def scores(self, q, k):
        """Differentiable (in proj_q / proj_k) block scores (B, H, Mb, Nb) fp32."""
        qi, ki = self._pool_input(q), self._pool_input(k)
        qb = ops.pool_blocks(qi, self.bq)
        kb = ops.pool_blocks(ki, self.bk) - ki.float().mean(-2, keepdim=True)
        if self.learnable:
            qb, kb = self.proj_q(qb), self.proj_k(kb)
        return (qb @ kb.transpose(-1, -2)) * (q.shape[-1] ** -0.5)

    @staticmethod
    def _pool_input(x):
        # fp32 and 16-bit inputs are pooled as given (the reference pools the
        # raw q / k); other dtypes go through fp32
        if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            x = x.float()
        return x.contiguous()

    def route(self, q, k, k_frac):
        """Hard top-k on the HIP kernels -> (lut (B,H,Mb,T) int32, T)."""
        pq = self.proj_q.weight if self.learnable else None
        pk = self.proj_k.weight if self.learnable else None
        with torch.no_grad():
            return ops.route_1d(self._pool_input(q), self._pool_input(k), k_frac, self.bq,
                                self.bk, pq, pk)

    def forward(self, q, k, k_frac, soft=False, need_mask=True):
        """Returns (mask, lut, topk, pc): mask (B,H,Mb,Nb) int8 hard mask (the soft
        mask when soft=True), lut (B,H,Mb,topk) int32, pc the block scores."""
        lut, topk = self.route(q, k, k_frac)
        pc = self.scores(q, k)
        if soft:
            return soft_topk(pc, k_frac, self.tau), lut, topk, pc
        mask = torch.zeros_like(pc, dtype=torch.int8).scatter_(-1, lut.long(), 1) \
            if need_mask else pc
        return mask, lut, topk, pc
