"""The DiT block around the SLA2 op (reference: models/imf_dit_video.py:121-187,
266-284, 422-532, 557-602): RMSNorm, SituAndMul / SwiGLUMlp, partial-RoPE MLA
attention with the output gate, and the vector-gated TransformerBlock.

Eager torch modules with the reference's names, arguments and parameter
names (state-dict compatible), so a block built here runs the training
forward (autograd) with any attn_impl of this package, e.g.
``functools.partial(SLA2CubeQATAttentionImpl, seq_len=L, num_heads=H, grid=...)``;
the fast forward-mode JVP of the same block is ``mla_jvp_fast.block_jvp``.
"""

import math
from functools import partial

import torch
import torch.nn as nn
import torch.nn.functional as F

__all__ = ["RMSNorm", "SituAndMul", "SwiGLUMlp", "MLAAttention", "TransformerBlock",
           "apply_rotary_pos_emb", "precompute_axial_rope_3d", "scaled_variance_linear",
           "sdpa_math_attention"]


def scaled_variance_linear(in_features, out_features, bias=True, init_constant=1.0):
    """nn.Linear with weights N(0, init_constant / sqrt(in_features))."""
    linear = nn.Linear(in_features, out_features, bias=bias)
    nn.init.normal_(linear.weight, std=init_constant / math.sqrt(in_features))
    if bias:
        nn.init.zeros_(linear.bias)
    return linear


def sdpa_math_attention(q, k, v):
    """Dense softmax attention on (b, l, H, hd) tensors (the default attn_impl)."""
    o = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    return o.transpose(1, 2)


class _RMSNormFunction(torch.autograd.Function):
    """RMSNorm on the GPU: one fused HIP kernel forward, one backward (plus the
    weight gradient's column sum); saves x only."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        from . import ops
        ctx.eps = eps
        ctx.save_for_backward(x, weight)
        return ops.rmsnorm_fwd(x, weight, eps)

    @staticmethod
    def backward(ctx, dy):
        from . import ops
        x, weight = ctx.saved_tensors
        dx, dw = ops.rmsnorm_bwd(dy, x, weight, ctx.eps)
        return dx, dw.to(weight.dtype), None


class RMSNorm(nn.Module):
    """Root mean square normalisation with fp32 accumulation.  GPU tensors (with
    an fp32 weight) run the fused kernels (sla2h_rmsnorm_fwd / _bwd); CPU
    tensors the eager expression."""

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        if (x.is_cuda and self.weight.dtype == torch.float32 and x.shape[-1] <= 1024
                and x.dtype in (torch.float32, torch.bfloat16, torch.float16)):
            return _RMSNormFunction.apply(x, self.weight, float(self.eps))
        xf = x.float()
        normed = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return normed.to(x.dtype) * self.weight


class _NormFanoutFunction(torch.autograd.Function):
    """RMSNorm of the fp32 residual stream for n linear consumers under
    autocast: one HIP kernel writes the normalised rows already rounded to the
    autocast dtype (what each consumer's cast would produce) and the function
    returns them as n outputs, one per consumer, plus x itself for its other
    use (the residual add).  The backward sums the consumers' 16-bit gradients
    in fp32 and adds the residual's gradient to dx in the same kernel."""

    @staticmethod
    def forward(ctx, x, weight, eps, n, dtype):
        from . import ops
        y = ops.rmsnorm_fwd16(x, weight, eps, dtype)
        ctx.eps = eps
        ctx.save_for_backward(x, weight)
        return (x.view_as(x), y) + tuple(y.view_as(y) for _ in range(n - 1))

    @staticmethod
    def backward(ctx, dpass, *dys):
        from . import ops
        x, weight = ctx.saved_tensors
        dys = [d for d in dys if d is not None]
        if not dys:
            return dpass, None, None, None, None
        dx, dw = ops.rmsnorm_bwd_sum(dys, x, weight, ctx.eps, dadd=dpass)
        return dx, dw.to(weight.dtype), None, None, None


def _norm_fanout(x, norm, n):
    """(x, n consumer inputs) of norm(x): the fused kernels when x is the fp32
    residual stream on the GPU under a 16-bit autocast, else (x, norm(x) n
    times)."""
    D = x.shape[-1]
    if (x.is_cuda and x.dtype == torch.float32 and torch.is_autocast_enabled("cuda")
            and norm.weight.dtype == torch.float32 and norm.weight.is_cuda
            and 8 <= D <= 512 and D & (D - 1) == 0 and x.is_contiguous()
            and x.data_ptr() % 16 == 0
            and torch.get_autocast_dtype("cuda") in (torch.bfloat16, torch.float16)):
        return _NormFanoutFunction.apply(x, norm.weight, float(norm.eps), n,
                                         torch.get_autocast_dtype("cuda"))
    y = norm(x)
    return (x,) + (y,) * n


class _GateMulFunction(torch.autograd.Function):
    """a * sigmoid(g) on 16-bit GPU tensors: one HIP kernel forward, one
    backward (sigmoid recomputed from g); saves a and g only."""

    @staticmethod
    def forward(ctx, a, g):
        from . import ops
        ctx.save_for_backward(a, g)
        return ops.gate_mul_fwd(a, g)

    @staticmethod
    def backward(ctx, dout):
        from . import ops
        a, g = ctx.saved_tensors
        return ops.gate_mul_bwd(dout, a, g)


def _gate_mul(a, g):
    """a * sigmoid(g): the fused kernels for 16-bit GPU tensors of one shape and
    dtype (16-byte aligned, a multiple of 8 elements), else the eager form."""
    if (a.is_cuda and g.is_cuda and a.dtype == g.dtype and a.shape == g.shape
            and a.dtype in (torch.bfloat16, torch.float16) and a.numel() % 8 == 0
            and a.is_contiguous() and g.is_contiguous()
            and a.data_ptr() % 16 == 0 and g.data_ptr() % 16 == 0):
        return _GateMulFunction.apply(a, g)
    return a * torch.sigmoid(g)


class _SituMulFunction(torch.autograd.Function):
    """SituAndMul on the GPU: one fused HIP kernel forward, one backward; saves
    only the inputs (the eager form keeps several fp32 intermediates)."""

    @staticmethod
    def forward(ctx, gate, up, beta, linear_beta):
        from . import ops
        ctx.beta, ctx.linear_beta = beta, linear_beta
        ctx.save_for_backward(gate, up)
        return ops.situ_mul_fwd(gate, up, beta, linear_beta)

    @staticmethod
    def backward(ctx, dh):
        from . import ops
        gate, up = ctx.saved_tensors
        dgate, dup = ops.situ_mul_bwd(dh, gate, up, ctx.beta, ctx.linear_beta)
        return dgate, dup, None, None


class SituAndMul(nn.Module):
    """situ(g) * up with situ(g) = beta tanh(g / beta) sigmoid(g); with
    linear_beta the up branch is soft-clamped to linear_beta tanh(up / linear_beta).
    GPU tensors of one 16-bit or fp32 dtype run the fused kernels
    (sla2h_situ_mul_fwd / _bwd); anything else (CPU tensors, mixed or other
    dtypes) the eager fp32 expression, each branch cast to fp32 on its own."""

    def __init__(self, beta=1.0, linear_beta=None):
        super().__init__()
        self.beta = beta
        self.linear_beta = linear_beta

    def forward(self, x, up=None):
        if up is None:
            d = x.shape[-1] // 2
            gate, up = x[..., :d], x[..., d:]
        else:
            gate = x
        if (gate.is_cuda and up.is_cuda and up.dtype == gate.dtype
                and gate.dtype in (torch.float16, torch.bfloat16, torch.float32)):
            return _SituMulFunction.apply(gate, up, float(self.beta),
                                          None if self.linear_beta is None
                                          else float(self.linear_beta))
        dtype = gate.dtype
        g, u = gate.float(), up.float()
        act = self.beta * torch.tanh(g / self.beta) * torch.sigmoid(g)
        if self.linear_beta is not None:
            u = self.linear_beta * torch.tanh(u / self.linear_beta)
        return (act * u).to(dtype)


class SwiGLUMlp(nn.Module):
    """Gated MLP w2(situ(w1 x) * w3 x)."""

    def __init__(self, in_features, hidden_features, weight_init_constant=1.0, situ_beta=1.0,
                 situ_linear_beta=None):
        super().__init__()
        linear = partial(scaled_variance_linear, bias=False, init_constant=weight_init_constant)
        self.w1 = linear(in_features, hidden_features)
        self.w3 = linear(in_features, hidden_features)
        self.w2 = linear(hidden_features, in_features)
        self.act = SituAndMul(beta=situ_beta, linear_beta=situ_linear_beta)

    def forward(self, x):
        return self._forward(x, x)

    def _forward(self, x1, x3):
        """The MLP with w1 reading x1 and w3 reading x3 (the same values)."""
        return self.w2(self.act(self.w1(x1), self.w3(x3)))


class _RopeFunction(torch.autograd.Function):
    """RoPE on the GPU: one HIP kernel forward (sla2h_rope), the inverse rotation
    of the output gradient backward."""

    @staticmethod
    def forward(ctx, x, rope_cos, rope_sin):
        from . import ops
        ctx.save_for_backward(rope_cos, rope_sin)
        return ops.rope(x, rope_cos, rope_sin)

    @staticmethod
    def backward(ctx, dout):
        from . import ops
        rope_cos, rope_sin = ctx.saved_tensors
        return ops.rope(dout.contiguous(), rope_cos, rope_sin, inverse=True), None, None


def apply_rotary_pos_emb(x, rope_cos, rope_sin):
    """Rotate channel pairs (x[..., 2i], x[..., 2i+1]) of x (b, l, H, hd) by the
    angles of rope_cos / rope_sin (l, hd // 2).  GPU tensors run the HIP kernel
    (sla2h_rope) forward and backward; CPU tensors the eager expression."""
    if (x.is_cuda and x.dim() == 4 and x.dtype in (torch.float32, torch.bfloat16, torch.float16)
            and rope_cos.dtype == torch.float32 and rope_sin.dtype == torch.float32):
        return _RopeFunction.apply(x, rope_cos, rope_sin)
    xf = x.float()
    re, im = xf[..., 0::2], xf[..., 1::2]
    c, s = rope_cos[None, :, None, :], rope_sin[None, :, None, :]
    out = torch.stack([re * c - im * s, re * s + im * c], dim=-1).flatten(-2)
    return out.to(x.dtype)


def precompute_axial_rope_3d(head_dim, grid_size, num_prefix_tokens, axis_dims=None,
                             theta=10000.0):
    """3-D axial RoPE angles: head_dim split over (t, h, w) (default ~1/4, 3/8,
    3/8, each even), standard 1-D RoPE per axis on the t-major patch grid; the
    prefix tokens come first with the identity rotation.
    Returns rope_cos, rope_sin: (num_prefix_tokens + T*Gh*Gw, head_dim // 2) fp32."""
    if axis_dims is None:
        dim_t = 2 * ((head_dim // 4) // 2)
        dim_h = 2 * (((head_dim - dim_t) // 2) // 2)
        axis_dims = (dim_t, dim_h, head_dim - dim_t - dim_h)
    assert sum(axis_dims) == head_dim and all(d % 2 == 0 for d in axis_dims)
    gt, gh, gw = grid_size
    pos = torch.meshgrid(torch.arange(gt, dtype=torch.float32),
                         torch.arange(gh, dtype=torch.float32),
                         torch.arange(gw, dtype=torch.float32), indexing="ij")
    parts = []
    for p, ad in zip(pos, axis_dims):
        freqs = 1.0 / (theta ** (torch.arange(0, ad, 2, dtype=torch.float32) / ad))
        parts.append(torch.outer(p.flatten(), freqs))
    angles = torch.cat([torch.zeros(num_prefix_tokens, head_dim // 2), torch.cat(parts, -1)], 0)
    return torch.cos(angles), torch.sin(angles)


class _AttnInFunction(torch.autograd.Function):
    """The (B, H, L, 64) fp16 operands of a tile-major SLA2 op straight from the
    sublayer's halves: q = [q_nope | q_rope], k = [k_nope | k_rope shared by
    the heads], v -- the reference's torch.cat and the op's permute + .half()
    in one HIP kernel per operand each way (sla2h_attn_in_fwd / _bwd)."""

    @staticmethod
    def forward(ctx, q_nope, q_rope, k_nope, k_rope, v):
        from . import ops
        H = q_nope.shape[2]
        ctx.meta = [(t.shape, t.dtype) for t in (q_nope, q_rope, k_nope, k_rope, v)]
        return (ops.attn_in_fwd((q_nope, q_rope), H), ops.attn_in_fwd((k_nope, k_rope), H),
                ops.attn_in_fwd((v[..., :32], v[..., 32:]), H))

    @staticmethod
    def backward(ctx, dqh, dkh, dvh):
        from . import ops
        grads = []
        for d, (lo, hi) in ((dqh, ctx.meta[0:2]), (dkh, ctx.meta[2:4])):
            if d is None:
                grads += [None, None]
                continue
            dlo = torch.empty(lo[0], device=d.device, dtype=lo[1])
            dhi = torch.empty(hi[0], device=d.device, dtype=hi[1])
            ops.attn_in_bwd(d, dlo, dhi)
            grads += [dlo, dhi]
        if dvh is None:
            grads.append(None)
        else:
            dv = torch.empty(ctx.meta[4][0], device=dvh.device, dtype=ctx.meta[4][1])
            ops.attn_in_bwd(dvh, dv[..., :32], dv[..., 32:])
            grads.append(dv)
        return tuple(grads)


class _AttnGateFunction(torch.autograd.Function):
    """round16(fp32(o) * sigmoid(g)) from a tile-major SLA2 op's fp16 output o
    (B, H, L, 64): the reference's permute / .to(float32) of o, its fp32 gate
    and the output projection's autocast cast in one HIP kernel each way
    (sla2h_attn_gate_fwd / _bwd); saves o and g only."""

    @staticmethod
    def forward(ctx, o, g):
        from . import ops
        ctx.save_for_backward(o, g)
        return ops.attn_gate_fwd(o, g)

    @staticmethod
    def backward(ctx, dy):
        from . import ops
        o, g = ctx.saved_tensors
        return ops.attn_gate_bwd(dy, o, g)


def _aligned16(*ts):
    return all(t.data_ptr() % 16 == 0 and all((st * t.element_size()) % 16 == 0
                                               for st in t.stride()[:-1]) and t.stride()[-1] == 1
               for t in ts)


def _tile_major_operands_ok(impl, q_nope, q_rope, k_nope, k_rope, v):
    """The fused operand path applies: the impl keeps the sequence tile-major
    and takes its operands directly (forward_tile_major), on GPU tensors with
    32-channel halves, 64-channel v, 16-bit rope / v and 16-byte accesses."""
    if not (getattr(impl, "pre_permuted", False) and hasattr(impl, "forward_tile_major")):
        return False
    ts = (q_nope, q_rope, k_nope, k_rope, v)
    half16 = (torch.float16, torch.bfloat16)
    return (all(t.is_cuda for t in ts) and q_nope.shape[-1] == 32 and q_rope.shape[-1] == 32
            and k_nope.shape[-1] == 32 and k_rope.shape[-1] == 32 and v.shape[-1] == 64
            and k_rope.shape[2] == 1 and q_nope.shape == q_rope.shape == k_nope.shape
            and q_nope.dtype in half16 + (torch.float32,) and k_nope.dtype in half16 + (torch.float32,)
            and q_rope.dtype in half16 and k_rope.dtype in half16 and v.dtype in half16
            and _aligned16(*ts))


class MLAAttention(nn.Module):
    """Multi-head latent attention with decoupled partial RoPE and the output
    gate.  q: d -> dq (RMSNorm) -> H (dn + dr); k/v: d -> [dc latent (RMSNorm) |
    dr shared rotary key] -> H (dn + dv); per-head RMSNorm on the nope bands;
    RoPE on the trailing dr channels (the key's band is shared by the heads);
    attn_impl(q, k, v) on (b, l, H, hd); output gate sigmoid(g_proj(x))."""

    def __init__(self, hidden_size, num_heads, q_lora_rank, kv_lora_rank, qk_nope_head_dim,
                 qk_rope_head_dim, v_head_dim, weight_init_constant=1.0, norm_eps=1e-6,
                 attn_impl=sdpa_math_attention, use_output_gate=True):
        super().__init__()
        self.hidden_size, self.num_heads = hidden_size, num_heads
        self.q_lora_rank, self.kv_lora_rank = q_lora_rank, kv_lora_rank
        self.qk_nope_head_dim, self.qk_rope_head_dim = qk_nope_head_dim, qk_rope_head_dim
        self.qk_head_dim = qk_nope_head_dim + qk_rope_head_dim
        self.v_head_dim = v_head_dim
        is_factory = isinstance(attn_impl, type) or (
            isinstance(attn_impl, partial) and isinstance(attn_impl.func, type))
        if is_factory:
            assert self.qk_head_dim == v_head_dim, (self.qk_head_dim, v_head_dim)
            attn_impl = attn_impl(self.qk_head_dim)
        self.attn_impl = attn_impl
        linear = partial(scaled_variance_linear, bias=False, init_constant=weight_init_constant)
        self.q_a_proj = linear(hidden_size, q_lora_rank)
        self.q_b_proj = linear(q_lora_rank, num_heads * self.qk_head_dim)
        self.kv_a_proj = linear(hidden_size, kv_lora_rank + qk_rope_head_dim)
        self.kv_b_proj = linear(kv_lora_rank, num_heads * (qk_nope_head_dim + v_head_dim))
        self.out_proj = linear(num_heads * v_head_dim, hidden_size)
        self.use_output_gate = use_output_gate
        if use_output_gate:
            self.g_proj = linear(hidden_size, num_heads * v_head_dim)
        self.q_a_layernorm = RMSNorm(q_lora_rank, eps=norm_eps)
        self.kv_a_layernorm = RMSNorm(kv_lora_rank, eps=norm_eps)
        self.q_norm = RMSNorm(qk_nope_head_dim, eps=norm_eps)
        self.k_norm = RMSNorm(qk_nope_head_dim, eps=norm_eps)

    def forward(self, x, rope_cos, rope_sin):
        return self._forward(x, x, x, rope_cos, rope_sin)

    def _forward(self, xq, xkv, xg, rope_cos, rope_sin):
        """The sublayer with q_a_proj, kv_a_proj and g_proj reading xq, xkv and
        xg (the same values)."""
        b, l, _ = xq.shape
        H = self.num_heads
        dn, dr, dv = self.qk_nope_head_dim, self.qk_rope_head_dim, self.v_head_dim
        q = self.q_b_proj(self.q_a_layernorm(self.q_a_proj(xq))).reshape(b, l, H, dn + dr)
        q_nope, q_rope = q.split([dn, dr], dim=-1)
        kv_latent, k_rope = self.kv_a_proj(xkv).split([self.kv_lora_rank, dr], dim=-1)
        kv = self.kv_b_proj(self.kv_a_layernorm(kv_latent)).reshape(b, l, H, dn + dv)
        k_nope, v = kv.split([dn, dv], dim=-1)
        q_nope, k_nope = self.q_norm(q_nope), self.k_norm(k_nope)
        q_rope = apply_rotary_pos_emb(q_rope, rope_cos, rope_sin)
        k_rope = apply_rotary_pos_emb(k_rope.unsqueeze(2), rope_cos, rope_sin)
        if _tile_major_operands_ok(self.attn_impl, q_nope, q_rope, k_nope, k_rope, v):
            # the op's fp16 tile-major operands straight from the halves, and
            # (under autocast) its output through the gate into the projection
            qh, kh, vh = _AttnInFunction.apply(q_nope, q_rope, k_nope, k_rope, v)
            o = self.attn_impl.forward_tile_major(qh, kh, vh)
            if self.use_output_gate:
                g = self.g_proj(xg)
                if (torch.is_autocast_enabled("cuda") and g.dtype == torch.get_autocast_dtype("cuda")
                        and g.dtype in (torch.float16, torch.bfloat16) and g.is_contiguous()
                        and g.data_ptr() % 16 == 0):
                    return self.out_proj(_AttnGateFunction.apply(o, g))
                attn = o.permute(0, 2, 1, 3).to(torch.promote_types(q_nope.dtype, q_rope.dtype))
                return self.out_proj(attn.reshape(b, l, H * dv) * torch.sigmoid(g))
            attn = o.permute(0, 2, 1, 3).to(torch.promote_types(q_nope.dtype, q_rope.dtype))
            return self.out_proj(attn.reshape(b, l, H * dv))
        k_rope = k_rope.expand(b, l, H, dr)
        q = torch.cat([q_nope, q_rope], dim=-1)
        k = torch.cat([k_nope, k_rope], dim=-1)
        attn = self.attn_impl(q, k, v).reshape(b, l, H * dv)
        if self.use_output_gate:
            attn = _gate_mul(attn, self.g_proj(xg))
        return self.out_proj(attn)


class _ResidualScaleFunction(torch.autograd.Function):
    """x + a * scale on the GPU: one HIP kernel forward, one backward (da and the
    scale gradient); the gradient of x is the output gradient itself."""

    @staticmethod
    def forward(ctx, x, a, scale):
        from . import ops
        ctx.save_for_backward(a, scale)
        return ops.residual_scale_fwd(x, a, scale)

    @staticmethod
    def backward(ctx, dy):
        from . import ops
        a, scale = ctx.saved_tensors
        da, ds = ops.residual_scale_bwd(dy, a, scale)
        return dy, da, ds.to(scale.dtype)


def _residual(x, a, scale):
    """x + a * scale.  The fused kernels take fp32 x, an a of x's shape on the
    same device and a (D,) fp32 scale (D = x.shape[-1]): they read scale[c]
    for every channel c.  Other operands (a broadcast scale, CPU tensors) run
    the eager expression."""
    if (x.is_cuda and a.is_cuda and scale.is_cuda and x.dtype == torch.float32
            and scale.dtype == torch.float32 and tuple(scale.shape) == (x.shape[-1],)
            and a.shape == x.shape and a.dtype in (torch.float32, torch.bfloat16, torch.float16)):
        return _ResidualScaleFunction.apply(x, a, scale)
    return x + a * scale


class TransformerBlock(nn.Module):
    """x += attn(norm1(x)) * attn_scale;  x += mlp(norm2(x)) * mlp_scale
    (vector gates initialised to zero)."""

    def __init__(self, hidden_size, num_heads, q_lora_rank, kv_lora_rank, qk_nope_head_dim,
                 qk_rope_head_dim, v_head_dim, mlp_ratio=8 / 3, weight_init_constant=1.0,
                 norm_eps=1e-6, attn_impl=sdpa_math_attention, use_attn_res=False, situ_beta=4.0,
                 situ_linear_beta=25.0, mla_use_output_gate=True):
        super().__init__()
        self.norm1 = RMSNorm(hidden_size, eps=norm_eps)
        self.attn = MLAAttention(hidden_size, num_heads=num_heads, q_lora_rank=q_lora_rank,
                                 kv_lora_rank=kv_lora_rank, qk_nope_head_dim=qk_nope_head_dim,
                                 qk_rope_head_dim=qk_rope_head_dim, v_head_dim=v_head_dim,
                                 weight_init_constant=weight_init_constant, norm_eps=norm_eps,
                                 attn_impl=attn_impl, use_output_gate=mla_use_output_gate)
        self.norm2 = RMSNorm(hidden_size, eps=norm_eps)
        self.mlp = SwiGLUMlp(hidden_size, int(hidden_size * mlp_ratio),
                             weight_init_constant=weight_init_constant, situ_beta=situ_beta,
                             situ_linear_beta=situ_linear_beta)
        self.attn_scale = nn.Parameter(torch.zeros(hidden_size))
        self.mlp_scale = nn.Parameter(torch.zeros(hidden_size))
        if use_attn_res:
            self.attn_res_norm = RMSNorm(hidden_size, eps=norm_eps)
            self.mlp_res_norm = RMSNorm(hidden_size, eps=norm_eps)
            self.attn_res_proj = scaled_variance_linear(hidden_size, 1, bias=False,
                                                        init_constant=weight_init_constant)
            self.mlp_res_proj = scaled_variance_linear(hidden_size, 1, bias=False,
                                                       init_constant=weight_init_constant)

    def forward(self, x, rope_cos, rope_sin):
        # each norm's output feeds several linears (three in the attention with
        # its output gate, two in the MLP); _norm_fanout hands each its own copy
        na = 3 if self.attn.use_output_gate else 2
        x, *n1 = _norm_fanout(x, self.norm1, na)
        if na == 2:
            n1.append(n1[0])
        x = _residual(x, self.attn._forward(*n1, rope_cos, rope_sin), self.attn_scale)
        x, n2a, n2b = _norm_fanout(x, self.norm2, 2)
        return _residual(x, self.mlp._forward(n2a, n2b), self.mlp_scale)
