"""SLA2 (sparse-linear attention) as an MLA attn_impl (reference:
models/sla2_attention.py:23-61).

The MLA module calls ``attn_impl(q, k, v)`` with (b, l, H, hd) tensors; this
wrapper permutes to (B, H, L, D), runs the SLA2 module (fp16 compute, no INT8,
query blocks of bq = 128 rows, key blocks of 64, per-(head, query-block)
alpha) on the gfx950 kernels, and permutes back.
"""

import math

import torch
import torch.nn as nn

from .sla2_vendor import SLA2


class SLA2AttentionImpl(nn.Module):
    """Stateful attn_impl: one SLA2 (router + alpha) per attention module.

    Args:
        head_dim: qk head dim D (= v head dim, 64).
        seq_len: full sequence length L; alpha_logit (H, ceil(L/bq)) is created
            here so an optimizer sees every parameter before the first step.
        num_heads: H.
        topk: routed fraction of key blocks.
        bq, bk: query / key block lengths (128 / 64).
        alpha_init: initial mixing ratio in (0, 1).
    """

    def __init__(self, head_dim, seq_len, num_heads, topk=0.03, bq=128, bk=64, alpha_init=0.9):
        super().__init__()
        self.seq_len = seq_len
        self.bq, self.bk, self.topk = bq, bk, topk
        self.sla2 = SLA2(head_dim, topk=topk, bq=bq, bk=bk, use_bf16=False, use_int8=False,
                         learnable_router=True, alpha_init=alpha_init, backend="triton")
        mb = math.ceil(seq_len / bq)
        init = torch.logit(torch.tensor(float(alpha_init)))
        self.sla2.alpha_logit = nn.Parameter(torch.full((num_heads, mb), init.item()))

    def forward(self, q, k, v):
        """q, k, v: (b, l, H, hd) -> (b, l, H, hd) attention output in q.dtype."""
        qh, kh, vh = (t.permute(0, 2, 1, 3) for t in (q, k, v))
        o = self.sla2(qh, kh, vh)
        return o.permute(0, 2, 1, 3).to(q.dtype)
