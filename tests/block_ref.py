"""Reference attention modules for the DiT-block parity tests (test code only).

Both mirror SLA2CubeQATAttentionImpl's interface, parameters and layout
(tokens to tile order, fp16, back), so that a TransformerBlock built with them
on the CPU runs the eager torch branches of every other layer:

  OracleCubeAttention  the CPU oracle's training forward / straight-through
                       backward (O.train_fwd / O.train_bwd) on a given LUT;
                       for small shapes.
  ForcedLutCubeAttention
                       the GPU op (ops.train_fwd / ops.train_bwd, validated
                       against the oracle on its own) on a given LUT, with
                       CPU tensors in and out; for full-size blocks, where
                       the oracle's attention would take minutes.

The LUT is the one the GPU block under test chose (captured by wrapping
route_tiles_fast), so that 16-bit rounding differences between the two
blocks' q / k cannot move a routing decision.
"""
import math

import torch
import torch.nn as nn

from oracle import sla2_oracle as O


class _OracleCubeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qh, kh, vh, alpha_logit, lut, Np, P):
        a = torch.sigmoid(alpha_logit.detach().float())
        fwd = O.train_fwd(qh, kh, vh, a, lut, Np, P, t16=torch.float16)
        ctx.save_for_backward(qh, kh, vh, a)
        ctx.fwd, ctx.lut, ctx.geom = fwd, lut, (Np, P)
        return fwd["o"]

    @staticmethod
    def backward(ctx, do):
        qh, kh, vh, a = ctx.saved_tensors
        Np, P = ctx.geom
        ref = O.train_bwd(qh, kh, vh, a, ctx.lut, Np, P, ctx.fwd, do.float(), t16=torch.float16)
        return ref["dq"], ref["dk"], ref["dv"], ref["d_alpha"], None, None, None


class _ForcedLutFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qh, kh, vh, alpha_logit, lut, Np, P):
        from imfvideo_amd import ops
        dev = torch.device("cuda")
        g = [t.to(dev, torch.float16).contiguous() for t in (qh, kh, vh)]
        a = torch.sigmoid(alpha_logit.detach().float()).to(dev)
        out = ops.train_fwd(*g, a, torch.as_tensor(lut).to(dev), Np)
        ctx.g, ctx.a, ctx.out = g, a, out
        return out["o"].float().cpu()

    @staticmethod
    def backward(ctx, do):
        from imfvideo_amd import ops
        dq, dk, dv, da = ops.train_bwd(*ctx.g, ctx.a, ctx.out, do.to("cuda"))
        return dq.float().cpu(), dk.float().cpu(), dv.float().cpu(), da.cpu(), None, None, None


class _CubeRef(nn.Module):
    FN = None

    def __init__(self, head_dim, seq_len, num_heads, grid, tile=(4, 4, 4), topk=0.03,
                 alpha_init=0.9, use_int8=True, pre_permuted=False, lut_source=None):
        super().__init__()
        from imfvideo_amd.mla_video_sparse_jvp import tile_permutation
        self.pre_permuted = pre_permuted
        E = tile[0] * tile[1] * tile[2]
        self.prefix_len = seq_len - grid[0] * grid[1] * grid[2]
        perm, inv, self.Np = tile_permutation(grid, tile, self.prefix_len, torch.device("cpu"))
        self.register_buffer("perm", perm, persistent=False)
        self.register_buffer("inv", inv, persistent=False)
        mb = self.Np + -(-self.prefix_len // E)
        self.proj_q = nn.Parameter(torch.eye(head_dim))
        self.proj_k = nn.Parameter(torch.eye(head_dim))
        self.alpha_logit = nn.Parameter(
            torch.full((num_heads, mb), math.log(alpha_init / (1 - alpha_init))))
        self.lut_source = lut_source

    def forward(self, q, k, v):
        def tm(x):
            x = x.permute(0, 2, 1, 3)
            if not self.pre_permuted:
                x = x[:, :, self.perm]
            return x.half().float()
        lut = self.lut_source()
        o = type(self).FN.apply(tm(q), tm(k), tm(v), self.alpha_logit, lut, self.Np,
                                self.prefix_len)
        if not self.pre_permuted:
            o = o[:, :, self.inv]
        return o.permute(0, 2, 1, 3).half().to(q.dtype)


class OracleCubeAttention(_CubeRef):
    FN = _OracleCubeFn


class ForcedLutCubeAttention(_CubeRef):
    FN = _ForcedLutFn


class LutRecorder:
    """Wraps a router function, keeping the LUTs it returns (as CPU tensors)."""

    def __init__(self, fn):
        self.fn = fn
        self.luts = []

    def __call__(self, *args, **kwargs):
        out = self.fn(*args, **kwargs)
        lut = out[0] if isinstance(out, tuple) else out
        self.luts.append(lut.detach().cpu())
        return out


def copy_block_to_cpu(blk, ref_blk):
    """Load the GPU block's parameters into the CPU reference block (same names)."""
    ref_blk.load_state_dict({k: v.detach().cpu() for k, v in blk.state_dict().items()},
                            strict=True)


def grad_report(gpu_blk, cpu_blk):
    """(name, gpu grad, cpu grad) for every parameter that has a gradient on
    either side."""
    cpu_p = dict(cpu_blk.named_parameters())
    out = []
    for n, p in gpu_blk.named_parameters():
        q = cpu_p[n]
        if p.grad is None and q.grad is None:
            continue
        assert p.grad is not None and q.grad is not None, n
        out.append((n, p.grad.detach().cpu(), q.grad.detach()))
    return out
