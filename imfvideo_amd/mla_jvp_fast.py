"""Forward-mode JVP of the MLA attention sublayer and the MLP sublayer around
the SLA2 op, on the gfx950 kernels (reference: models/mla_jvp_fast.py:53-228,
models/triton_mla_block_jvp.py:585-617, 813-850).

(primal, tangent) pairs propagate by hand as stacked rows [primal; tangent]
(M = 2*B*S): the GEMMs run once over both halves on hipBLASLt (fp16 in,
fp32 accumulate, fp16 out), the RMSNorm / RoPE / gate / SituAndMul JVP
stages are HIP row kernels (include/sla2h.h), and the attention op is one of
the SLA2 JVP ops of this package:

  p["cube"]  sla2_cube_qat_jvp_fused (tile-major; q/k/v are written at their
             tile positions directly and read back from them)
  p["sla2"]  route_blocks + sla2_mla_jvp (1-D blocks)
  neither    dense softmax attention JVP, as the 1-D op with every key block
             routed and alpha = 1

Shapes: h, dh (b, l, d) fp32; H heads, q/kv latent ranks dq/dc, nope / rope /
value head dims dn = dr = 32, dv = 64.
"""

import torch
import torch.nn.functional as F

from . import _lib, ops
from .sla2_cube_qat import sla2_cube_qat_jvp_fused
from .sla2_mla_jvp import _sla2_mla_jvp, route_blocks, sla2_mla_jvp

__all__ = ["mla_params_from_block", "mla_fp16_cache", "attn_sublayer_jvp", "mlp_sublayer_jvp",
           "block_jvp", "pack_block", "build_fast_jvp_state"]

_FP16 = torch.float16
_F32_CODE = 2


def mla_params_from_block(block):
    """Parameter dict of an imf_dit_video.TransformerBlock (reference
    models/triton_mla_block_jvp.py:813-850): weights detached, fp32."""
    attn = block.attn
    return {
        "w_norm1": block.norm1.weight.detach(), "w_qa": attn.q_a_proj.weight.detach(),
        "w_kva": attn.kv_a_proj.weight.detach(), "w_qa_ln": attn.q_a_layernorm.weight.detach(),
        "w_kva_ln": attn.kv_a_layernorm.weight.detach(), "w_qb": attn.q_b_proj.weight.detach(),
        "w_kvb": attn.kv_b_proj.weight.detach(), "w_qnorm": attn.q_norm.weight.detach(),
        "w_knorm": attn.k_norm.weight.detach(), "w_out": attn.out_proj.weight.detach(),
        "g_attn": block.attn_scale.detach(), "w_norm2": block.norm2.weight.detach(),
        "w_gate": block.mlp.w1.weight.detach(), "w_up": block.mlp.w3.weight.detach(),
        "w_down": block.mlp.w2.weight.detach(), "g_mlp": block.mlp_scale.detach(),
        "situ_beta": getattr(getattr(block.mlp, "act", None), "beta", 1.0),
        "w_og": attn.g_proj.weight.detach() if getattr(attn, "use_output_gate", False) else None,
        "H": attn.num_heads, "dq": attn.q_lora_rank, "dc": attn.kv_lora_rank,
        "dn": attn.qk_nope_head_dim, "dr": attn.qk_rope_head_dim, "dv": attn.v_head_dim,
    }


def mla_fp16_cache(p):
    """fp16 GEMM weights (N, K): w_a = [w_qa; w_kva] fused, w_qb, w_kvb, w_out,
    w_gate_up = [w_gate; w_up], w_down, and w_og when the output gate is on."""
    w = {"w_a": torch.cat([p["w_qa"], p["w_kva"]], 0), "w_qb": p["w_qb"], "w_kvb": p["w_kvb"],
         "w_out": p["w_out"], "w_gate_up": torch.cat([p["w_gate"], p["w_up"]], 0),
         "w_down": p["w_down"]}
    if p.get("w_og") is not None:
        w["w_og"] = p["w_og"]
    return {k: v.detach().to(_FP16).contiguous() for k, v in w.items()}


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _rms(x, dx, w, rows, D, sx, y, dy, sy, eps):
    """RMSNorm JVP rows: x/dx fp32 or fp16 views (row stride sx), into y/dy."""
    code = lambda t: _F32_CODE if t.dtype == torch.float32 else ops._dtype_code(t)
    _lib.check(_lib.load().sla2h_rmsnorm_jvp(
        x.data_ptr(), dx.data_ptr(), code(x), w.data_ptr(), rows, D, sx, y.data_ptr(),
        dy.data_ptr(), sy, code(y), float(eps), _stream(x.device)), "sla2h_rmsnorm_jvp")


def _vec(w, dev):
    return w.detach().to(dev, torch.float32).contiguous()


def attn_sublayer_jvp(h, dh, p, w16, cos, sin, eps, stage_events=None):
    """MLA attention sublayer JVP: a = out_proj(gate(attn(norm1(h)))) * g_attn.

    Returns (a, da): (b, l, d) fp32.  stage_events: optional three HIP events
    recorded before the attention op, after it, and at the end.
    """
    proj = _attn_sublayer_proj(h, dh, p, w16, cos, sin, eps, stage_events)
    # fp16 GEMM output times the fp32 gain: one kernel (fp32 by type promotion)
    out = proj * _vec(p["g_attn"], h.device)
    if stage_events:
        stage_events[2].record()
    B = h.shape[0]
    return out[:B], out[B:]


def _attn_sublayer_proj(h, dh, p, w16, cos, sin, eps, stage_events=None):
    """The attention sublayer JVP up to its output projection: the fp16 GEMM
    output (2b, l, d), rows [primal; tangent], before the gain g_attn."""
    rec = (lambda i: stage_events[i].record()) if stage_events else (lambda i: None)
    ops._need_gpu(h, dh)
    B, S, D = h.shape
    H, dq, dc = p["H"], p["dq"], p["dc"]
    dn, dr, dv = p["dn"], p["dr"], p["dv"]
    if (dn, dr, dv) != (32, 32, 64):
        raise ValueError(f"built for dn = dr = 32, dv = 64; got {(dn, dr, dv)}")
    dev = h.device
    half = B * S
    M = 2 * half
    h, dh = h.float().contiguous(), dh.float().contiguous()

    xs = torch.empty(M, D, device=dev, dtype=_FP16)                   # [n1; dn1]
    _rms(h, dh, _vec(p["w_norm1"], dev), half, D, D, xs[:half], xs[half:], D, eps)
    a_ = F.linear(xs, w16["w_a"])                                     # (M, dq+dc+dr)
    wa = dq + dc + dr
    q_lat = torch.empty(M, dq, device=dev, dtype=_FP16)
    _rms(a_, a_[half:], _vec(p["w_qa_ln"], dev), half, dq, wa, q_lat, q_lat[half:], dq, eps)
    kv_lat = torch.empty(M, dc, device=dev, dtype=_FP16)
    _rms(a_[:, dq:], a_[half:, dq:], _vec(p["w_kva_ln"], dev), half, dc, wa, kv_lat,
         kv_lat[half:], dc, eps)
    qb = F.linear(q_lat, w16["w_qb"])                                 # (M, H*(dn+dr))
    kvb = F.linear(kv_lat, w16["w_kvb"])                              # (M, H*(dn+dv))

    cube = p.get("cube")
    pos = None
    if cube is not None and not cube.get("pre_permuted", False):
        pos = cube["inv"].to(dev, torch.int32).contiguous()
    qkv = [torch.empty(B, H, S, 64, device=dev, dtype=_FP16) for _ in range(6)]
    kr = a_[:, dq + dc:]
    _lib.check(_lib.load().sla2h_mla_qkv_prep(
        qb.data_ptr(), kvb.data_ptr(), kr.data_ptr(), wa, _vec(p["w_qnorm"], dev).data_ptr(),
        _vec(p["w_knorm"], dev).data_ptr(), cos.float().contiguous().data_ptr(),
        sin.float().contiguous().data_ptr(), ops._ptr(pos), 0, B, S, H, dn, dr, dv, float(eps),
        *(t.data_ptr() for t in qkv), _stream(dev)), "sla2h_mla_qkv_prep")
    q, dq_, k, dk, v, dv_ = qkv
    rec(0)

    if cube is not None:
        o, do = sla2_cube_qat_jvp_fused(q, k, v, dq_, dk, dv_, cube["alpha"], cube["topk"],
                                        cube["Np"], cube["E"], cube["P"],
                                        proj_q=cube.get("proj_q"), proj_k=cube.get("proj_k"))
    elif "sla2" in p:
        sl = p["sla2"]
        lut, T = route_blocks(q, k, sl["topk"], sl["bq"], sl["bk"], proj_q=sl.get("proj_q"),
                              proj_k=sl.get("proj_k"))
        # the LUT comes straight from route_blocks: no range check (a host sync)
        o, do = _sla2_mla_jvp(q, k, v, dq_, dk, dv_, sl["alpha"], sl["topk"], sl["bq"], sl["bk"],
                              lut, T, 64, False)
    else:  # dense softmax attention: every key block routed, alpha = 1
        nb = -(-S // 64)
        mq = -(-S // 64)
        lut = torch.arange(nb, device=dev, dtype=torch.int32).view(1, 1, 1, nb).expand(
            B, H, mq, nb).contiguous()
        o, do = ops.jvp_1d(q, k, v, dq_, dk, dv_, torch.ones(H, mq, device=dev), lut, 64)

    rec(1)
    w_og = w16.get("w_og")
    z = F.linear(xs, w_og) if w_og is not None else None             # (M, H*dv)
    gated = torch.empty(M, H * dv, device=dev, dtype=_FP16)
    _lib.check(_lib.load().sla2h_mla_out_gate(
        o.data_ptr(), do.data_ptr(), ops._ptr(pos), ops._ptr(z), 0, B, S, H, dv,
        gated.data_ptr(), _stream(dev)), "sla2h_mla_out_gate")
    return F.linear(gated, w16["w_out"]).view(2 * B, S, D)


def mlp_sublayer_jvp(h, dh, p, w16, eps):
    """MLP sublayer JVP: m = down(situ(gate_up(norm2(h)))) * g_mlp -> (m, dm) fp32.
    As in the reference's fast JVP, the up branch is not soft-clamped (the
    eager SwiGLUMlp's linear_beta is ignored here)."""
    dwn = _mlp_sublayer_proj(h, dh, p, w16, eps) * _vec(p["g_mlp"], h.device)
    B = h.shape[0]
    return dwn[:B], dwn[B:]


def _mlp_sublayer_proj(h, dh, p, w16, eps):
    """The MLP sublayer JVP up to its down projection: the fp16 GEMM output
    (2b, l, d), rows [primal; tangent], before the gain g_mlp."""
    ops._need_gpu(h, dh)
    B, S, D = h.shape
    dev = h.device
    half = B * S
    M = 2 * half
    h, dh = h.float().contiguous(), dh.float().contiguous()
    xs = torch.empty(M, D, device=dev, dtype=_FP16)
    _rms(h, dh, _vec(p["w_norm2"], dev), half, D, D, xs[:half], xs[half:], D, eps)
    gu = F.linear(xs, w16["w_gate_up"])                               # (M, 2F)
    f = gu.shape[1] // 2
    act = torch.empty(M, f, device=dev, dtype=_FP16)
    _lib.check(_lib.load().sla2h_situ_jvp(gu.data_ptr(), half, f, float(p.get("situ_beta", 1.0)),
                                          0, act.data_ptr(), _stream(dev)), "sla2h_situ_jvp")
    return F.linear(act, w16["w_down"]).view(2 * B, S, D)


def pack_block(block, tile_major=False):
    """(params, fp16 weight cache) of one TransformerBlock for the fast JVP
    (the inner pack of models/mla_jvp_fast.py:252-300): the block parameters,
    the attention-residual heads when the block has them, and a snapshot of the
    attention's routing / mixing state so that the fast path computes the
    training forward's attention function --
      cube (SLA2CubeQATAttentionImpl): alpha = sigmoid(alpha_logit) (H, Mb),
        proj_q, proj_k, topk, Np, E, P (prefix tokens), perm, inv and
        pre_permuted = tile_major (the model keeps tokens tile-major);
      sla2 (SLA2AttentionImpl): alpha (H, Mb), the router projections, topk, bq, bk.
    Rebuild after every optimizer step (the weights change)."""
    p = mla_params_from_block(block)
    for name in ("attn_res_norm", "mlp_res_norm"):
        if hasattr(block, name):
            p[name] = getattr(block, name).weight.detach()
    for name in ("attn_res_proj", "mlp_res_proj"):
        if hasattr(block, name):
            p[name] = getattr(block, name).weight.detach()
    impl = getattr(block.attn, "attn_impl", None)
    if isinstance(impl, torch.nn.Module) and hasattr(impl, "perm"):
        p["cube"] = {
            "pre_permuted": bool(tile_major),
            "alpha": torch.sigmoid(impl.alpha_logit.detach()).float(),
            "proj_q": impl.proj_q.detach(), "proj_k": impl.proj_k.detach(),
            "topk": impl.topk_frac, "Np": impl.Np, "E": impl.E, "P": impl.prefix_len,
            "perm": impl.perm, "inv": impl.inv,
        }
    elif isinstance(impl, torch.nn.Module) and hasattr(impl, "sla2"):
        sl = impl.sla2
        if sl.alpha_logit is None:
            raise ValueError("SLA2 alpha is created by the first forward; run the block once")
        p["sla2"] = {
            "alpha": torch.sigmoid(sl.alpha_logit.detach()).float(),
            "proj_q": sl.router.proj_q.weight.detach(), "proj_k": sl.router.proj_k.weight.detach(),
            "topk": impl.topk, "bq": impl.bq, "bk": impl.bk,
        }
    return p, mla_fp16_cache(p)


def build_fast_jvp_state(net):
    """Per-block (params, fp16 cache) of a DiT's shared trunk and u-heads plus
    the u-branch output tensors (models/mla_jvp_fast.py:252-316); net needs
    the reference model's attributes (shared_blocks, u_heads, u_out_res_norm /
    _proj, u_final_layer, rope_cos / rope_sin, rmsnorm_eps,
    attn_res_block_size, prefix_tokens, tile_major)."""
    tm = getattr(net, "tile_major", False)
    return {
        "shared": [pack_block(b, tm) for b in net.shared_blocks],
        "u_heads": [pack_block(b, tm) for b in net.u_heads],
        "u_out_res": (net.u_out_res_norm.weight.detach(), net.u_out_res_proj.weight.detach()),
        "u_final": (net.u_final_layer.norm.weight.detach(),
                    net.u_final_layer.linear.weight.detach(),
                    net.u_final_layer.linear.bias.detach()),
        "rope": (net.rope_cos, net.rope_sin),
        "eps": net.rmsnorm_eps,
        "bs": net.attn_res_block_size,
        "prefix_tokens": net.prefix_tokens,
    }


def block_jvp(h, dh, p, w16, cos, sin, eps):
    """TransformerBlock JVP: x += attn sublayer; x += MLP sublayer -> (x, dx) fp32.
    Each residual update x + proj * g is one HIP kernel per half (the gain's
    product and the sum rounded separately, as the two torch operations
    would), reading the sublayer's fp16 GEMM output directly."""
    h, dh = h.float().contiguous(), dh.float().contiguous()
    B = h.shape[0]
    dev = h.device
    a = _attn_sublayer_proj(h, dh, p, w16, cos, sin, eps)
    g = _vec(p["g_attn"], dev)
    h, dh = ops.residual_scale_fwd(h, a[:B], g), ops.residual_scale_fwd(dh, a[B:], g)
    m = _mlp_sublayer_proj(h, dh, p, w16, eps)
    g = _vec(p["g_mlp"], dev)
    return ops.residual_scale_fwd(h, m[:B], g), ops.residual_scale_fwd(dh, m[B:], g)


# reference-private names (models/mla_jvp_fast.py:53, 198)
_attn_sublayer_jvp = attn_sublayer_jvp
_mlp_sublayer_jvp = mlp_sublayer_jvp
_mla_fp16_cache = mla_fp16_cache
