"""INT8 block quantisation entry point with the reference's name and signature.

Mirrors ``quantize_qkv`` of models/sla2_vendor/kernel_sparse_qat.py:144-151:
per (b, h, BLOCK_L-token block) symmetric INT8 with
``s = max|x| / 127 + 1e-12`` and ``q = round_half_away(x / s)``, computed by
the gfx950 kernel behind ``sla2h_quantize``.
"""

import torch

from . import ops

__all__ = ["quantize_qkv"]


def quantize_qkv(x, BLOCK_L):
    """x: (B,H,L,D) 16-bit -> (xq int8 (B,H,L,D), xs fp32 (B,H,ceil(L/BLOCK_L))).

    fp32 inputs are first rounded to bfloat16 (the 16-bit type of this build);
    the reference quantises from fp16 copies.
    """
    if x.dtype not in (torch.float16, torch.bfloat16):
        x = x.to(torch.bfloat16)
    return ops.quantize(x, BLOCK_L)
