"""Full-size GPU parity runs of BASELINE Configs 2, 4 and 5 (marked gpu).

Config 2: the op forward only at (1, 8, 29952, 64); INT8 operands, scales and
  the LUT bit-exact on every head, o against the oracle on every head at the
  north star's unscaled max-abs 2e-2.
Config 4: the MLA attention sublayer JVP at d=512, H=8, dq=256, dc=128,
  dn=dr=32, dv=64, partial axial RoPE over the 12x48x52 grid (the inputs of
  bench.py --config 4), on the 1-D SLA2 path the bench measures and on the
  cube path; the oracle's attention takes the GPU's LUT, so 16-bit GEMM
  rounding cannot move a routing decision.
Config 5: (a) the attention op's training step at B=2 (fp16 as the module
  casts), LUT bit-exact on every head, forward and straight-through
  gradients against the oracle on every head; (b) one DiT block (d=512, H=8,
  MLP ratio 4, ReZero scales 0.1, tile-major residency) forward + backward at
  B=2 x 29952 tokens: output, input gradient and every parameter gradient
  against the same block run eagerly on the CPU, whose attention is the
  oracle's training forward / straight-through backward fed the same LUT;
  (c) the block's fast JVP (block_jvp from its pack_block snapshot) at B=2
  against the oracle restatement.
"""
import math
from functools import partial

import numpy as np
import pytest
import torch

from oracle import sla2_oracle as O
from tests.block_ref import LutRecorder, OracleCubeAttention, copy_block_to_cpu, grad_report
from tests.helpers import make_inputs, max_abs, rel_l2
from tests.test_gpu_parity import TOL_MAX, TOL_REL, config_inputs, cuda, run_full, say

pytestmark = pytest.mark.gpu
GRID = (12, 48, 52)
S_FULL = 29952


def _check(got, want, tag, rel=TOL_REL, mx=TOL_MAX, unscaled=False):
    """Max-abs against mx scaled by the reference's peak (|want| up to ~10 for
    the block and sublayer outputs; the gradients scale with their inputs) and
    rel-L2; unscaled=True also asserts the plain max-abs mx, the north star's
    bound for the op's own outputs.  Both figures are printed."""
    got, want = got.detach().cpu().double(), want.detach().cpu().double()
    bound = mx * max(1.0, want.abs().max().item())
    r = rel_l2(got, want)
    m = max_abs(got, want)
    print(f"  {tag}: max {m:.2e} (unscaled bound {mx:.0e}, scaled {bound:.2e}) rel {r:.2e}",
          flush=True)
    assert torch.isfinite(got).all(), tag
    assert m < bound and r < rel, tag
    if unscaled:
        assert m < mx, tag


# ---------------------------------------------------------------------------
# Config 2
# ---------------------------------------------------------------------------
def test_config2_full_size_forward():
    say("config2 full size forward (1,8,29952,64)")
    ins, Np, P = config_inputs(3)
    prim = {n: ins[n] for n in ("q", "k", "v")}
    alpha = torch.full((8, Np), 0.9)
    o, do, aux = run_full(prim, alpha, 0.1, Np, P, tangent=False)
    assert do is None and torch.isfinite(o).all()
    f = {n: t.float() for n, t in prim.items()}
    q8, qs = O.quantize_blocks(f["q"])
    k8, ks = O.quantize_blocks(f["k"])
    assert np.array_equal(aux["q8"].numpy(), q8) and np.array_equal(aux["qs"].numpy(), qs)
    assert np.array_equal(aux["k8"].numpy(), k8) and np.array_equal(aux["ks"].numpy(), ks)
    lut, T, _, _ = O.route(f["q"], f["k"], 0.1, Np, P)
    assert T == 46 and np.array_equal(aux["lut"].numpy(), lut)
    for h in range(8):  # every head, at the north star's unscaled bound
        sl = slice(h, h + 1)
        eo, edo = O.cube_jvp(f["q"][:, sl], f["k"][:, sl], f["v"][:, sl], None, None, None,
                             alpha[sl], lut[:, sl], Np, P,
                             quant=(q8[:, sl], qs[:, sl], k8[:, sl], ks[:, sl]))
        assert edo is None
        _check(o[:, sl], eo, f"head {h} o", unscaled=True)


# ---------------------------------------------------------------------------
# Config 4: the MLA attention sublayer JVP (bench.py --config 4 inputs)
# ---------------------------------------------------------------------------
def mla_config4_inputs():
    """The parameters and inputs of bench.py's mla_bench, drawn in the same
    order from the same seed, on the CPU."""
    B, S, D, H, dq, dc = 1, S_FULL, 512, 8, 256, 128
    g = torch.Generator().manual_seed(4)
    lin = lambda o, i: torch.randn(o, i, generator=g) * 0.5 / math.sqrt(i)
    ones = torch.ones
    p = {"H": H, "dq": dq, "dc": dc, "dn": 32, "dr": 32, "dv": 64, "w_norm1": ones(D),
         "w_qa": lin(dq, D), "w_kva": lin(dc + 32, D), "w_qa_ln": ones(dq), "w_kva_ln": ones(dc),
         "w_qb": lin(H * 64, dq), "w_kvb": lin(H * 96, dc), "w_qnorm": ones(32),
         "w_knorm": ones(32), "w_out": lin(D, H * 64), "g_attn": ones(D), "w_og": lin(H * 64, D),
         "w_norm2": ones(D), "w_gate": lin(8, D), "w_up": lin(8, D), "w_down": lin(D, 8),
         "g_mlp": ones(D)}
    x = torch.randn(B, S, D, generator=g).to(torch.bfloat16).float()
    dx = 0.1 * torch.randn(B, S, D, generator=g)
    return p, x, dx


@pytest.mark.parametrize("path", ["sla2", "cube"])
def test_config4_full_size(path, monkeypatch):
    say("config4 MLA sublayer JVP full size, path", path)
    from imfvideo_amd import ops
    from imfvideo_amd.imf_dit_video import precompute_axial_rope_3d
    from imfvideo_amd.mla_jvp_fast import attn_sublayer_jvp, mla_fp16_cache
    from imfvideo_amd.mla_video_sparse_jvp import tile_permutation
    p, x, dx = mla_config4_inputs()
    H = p["H"]
    cos, sin = precompute_axial_rope_3d(32, GRID, 0, axis_dims=(8, 12, 12))
    pg = {k: (cuda(v) if torch.is_tensor(v) else v) for k, v in p.items()}
    if path == "sla2":
        alpha = torch.full((H, -(-S_FULL // 128)), 0.9)
        pg["sla2"] = {"alpha": cuda(alpha), "proj_q": None, "proj_k": None, "topk": 0.1,
                      "bq": 128, "bk": 64}
    else:
        perm, inv, Np = tile_permutation(GRID, (4, 4, 4), 0, torch.device("cpu"))
        g = torch.Generator().manual_seed(41)
        alpha = torch.rand(H, Np, generator=g) * 0.8 + 0.1
        pg["cube"] = {"alpha": cuda(alpha), "topk": 0.1, "Np": Np, "E": 64, "P": 0,
                      "perm": perm, "inv": inv}
    rec = LutRecorder(ops.route_topk)
    monkeypatch.setattr(ops, "route_topk", rec)
    a, da = attn_sublayer_jvp(cuda(x), cuda(dx), pg, mla_fp16_cache(pg), cuda(cos), cuda(sin),
                              1e-6)
    torch.cuda.synchronize()
    assert len(rec.luts) == 1
    lut = rec.luts[0].numpy()
    if path == "sla2":
        assert lut.shape == (1, H, 234, 46)
        ref_attn = lambda q, k, v, dq, dk, dv: O.jvp_1d(q, k, v, dq, dk, dv, alpha, lut, 128)
    else:
        assert lut.shape == (1, H, 468, 46)

        def ref_attn(q, k, v, dq, dk, dv):
            t = lambda y: y[:, :, perm]
            o, do = O.cube_jvp(*(t(y) for y in (q, k, v, dq, dk, dv)), alpha, lut, Np, 0,
                               t16=torch.float16)
            return o[:, :, inv], do[:, :, inv]
    want_a, want_da = O.mla_attn_jvp(x, dx, p, cos, sin, 1e-6, ref_attn)
    _check(a, want_a, f"{path} a")
    _check(da, want_da, f"{path} da")


# ---------------------------------------------------------------------------
# Config 5
# ---------------------------------------------------------------------------
def test_config5_attention_op_training_step():
    say("config5 attention op training step (2,8,29952,64) fp16")
    from imfvideo_amd import ops
    B, H, Np = 2, 8, 468
    q, k, v = make_inputs(5, B, H, S_FULL, dtype=torch.float16, rms_qk=True, tangent=False)
    gdo = torch.Generator().manual_seed(55)
    do = torch.randn(B, H, S_FULL, 64, generator=gdo).half()
    g = torch.Generator().manual_seed(56)
    alpha = torch.rand(H, Np, generator=g) * 0.8 + 0.1
    gq, gk, gv = cuda(q), cuda(k), cuda(v)
    _, _, _, _, qpool, kpool_t = ops.quant_pool_qk(gq, gk, Np)
    lut = ops.route_topk(qpool, kpool_t, 46, 0.125)
    out = ops.train_fwd(gq, gk, gv, cuda(alpha), lut, Np)
    dq, dk, dv, da = ops.train_bwd(gq, gk, gv, cuda(alpha), out, cuda(do))
    torch.cuda.synchronize()
    f = {"q": q.float(), "k": k.float(), "v": v.float()}
    want_lut, T, _, _ = O.route(f["q"], f["k"], 0.1, Np, 0)
    assert np.array_equal(lut.cpu().numpy(), want_lut)
    for h in range(H):  # every head
        sl = slice(h, h + 1)
        fh = {n: t[:, sl] for n, t in f.items()}
        ref = O.train_fwd(fh["q"], fh["k"], fh["v"], alpha[sl], want_lut[:, sl], Np, 0,
                          t16=torch.float16)
        for n in ("o", "o_s", "o_l", "qphi"):
            _check(out[n][:, sl].float(), ref[n], f"h{h} {n}")
        _check(out["lse"][:, sl], ref["lse"], f"h{h} lse", rel=1e-5)
        fwd = {n: out[n][:, sl].cpu().float() for n in ("o_s", "o_l", "lse", "den", "qphi",
                                                        "htot", "ztot")}
        rb = O.train_bwd(fh["q"], fh["k"], fh["v"], alpha[sl], want_lut[:, sl], Np, 0, fwd,
                         do[:, sl].float(), t16=torch.float16)
        for t_, n in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
            _check(t_[:, sl].float(), rb[n], f"h{h} {n}")
        _check(da[sl], rb["d_alpha"], f"h{h} d_alpha")


def _config5_block(dev, attn_cls, **extra):
    from imfvideo_amd.imf_dit_video import TransformerBlock
    impl = partial(attn_cls, seq_len=S_FULL, num_heads=8, grid=GRID, tile=(4, 4, 4), topk=0.1,
                   pre_permuted=True, **extra)
    blk = TransformerBlock(512, 8, 256, 128, 32, 32, 64, mlp_ratio=4, weight_init_constant=0.5,
                           attn_impl=impl)
    with torch.no_grad():
        blk.attn_scale.fill_(0.1)
        blk.mlp_scale.fill_(0.1)
    return blk.to(dev)


def _config5_rope():
    from imfvideo_amd.imf_dit_video import precompute_axial_rope_3d
    from imfvideo_amd.mla_video_sparse_jvp import tile_permutation
    perm, _, _ = tile_permutation(GRID, (4, 4, 4), 0, torch.device("cpu"))
    cos, sin = precompute_axial_rope_3d(32, GRID, 0, axis_dims=(8, 12, 12))
    return cos[perm].contiguous(), sin[perm].contiguous()


def test_config5_block_forward_backward(monkeypatch):
    say("config5 DiT block forward + backward, B=2 x 29952, d=512, H=8")
    import imfvideo_amd.sla2_cube_qat as cq
    torch.manual_seed(5)
    blk = _config5_block("cuda", cq.SLA2CubeQATAttentionImpl)
    with torch.no_grad():  # non-uniform mixing so the alpha gradient is exercised
        a = blk.attn.attn_impl.alpha_logit
        a.add_(torch.linspace(-1, 1, a.numel(), device="cuda").view_as(a))
    rec = LutRecorder(cq.route_tiles_fast)
    monkeypatch.setattr(cq, "route_tiles_fast", rec)
    cos, sin = _config5_rope()
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, S_FULL, 512, generator=g).to(torch.bfloat16).float()
    w = torch.randn(2, S_FULL, 512, generator=g)
    xg = cuda(x).requires_grad_()
    out = blk(xg, cuda(cos), cuda(sin))
    (out * cuda(w)).sum().backward()
    torch.cuda.synchronize()
    assert len(rec.luts) == 1
    say("  cpu eager block")
    ref = _config5_block("cpu", OracleCubeAttention, lut_source=lambda: rec.luts[0])
    copy_block_to_cpu(blk, ref)
    xc = x.clone().requires_grad_()
    out_ref = ref(xc, cos, sin)
    (out_ref * w).sum().backward()
    _check(out, out_ref, "out")
    _check(xg.grad, xc.grad, "x.grad")
    for name, got, want in grad_report(blk, ref):
        _check(got, want, f"grad {name}")


def test_config5_block_jvp(monkeypatch):
    say("config5 block_jvp (pack_block snapshot, tile-major), B=2 x 29952")
    from imfvideo_amd import ops
    from imfvideo_amd.mla_jvp_fast import block_jvp, pack_block
    import imfvideo_amd.sla2_cube_qat as cq
    torch.manual_seed(7)
    blk = _config5_block("cuda", cq.SLA2CubeQATAttentionImpl)
    pk, w16 = pack_block(blk, tile_major=True)
    assert pk["cube"]["pre_permuted"] is True
    cos, sin = _config5_rope()
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, S_FULL, 512, generator=g).to(torch.bfloat16).float()
    dx = 0.1 * torch.randn(2, S_FULL, 512, generator=g)
    rec = LutRecorder(ops.route_topk)
    monkeypatch.setattr(ops, "route_topk", rec)
    y, dy = block_jvp(cuda(x), cuda(dx), pk, w16, cuda(cos), cuda(sin), 1e-6)
    torch.cuda.synchronize()
    assert len(rec.luts) == 1
    lut = rec.luts[0].numpy()
    pc = {k_: (v_.detach().cpu().float() if torch.is_tensor(v_) else v_) for k_, v_ in pk.items()
          if k_ != "cube"}
    alpha = pk["cube"]["alpha"].cpu()
    ref_attn = lambda q, k, v, dq, dk, dv: O.cube_jvp(q, k, v, dq, dk, dv, alpha, lut, 468, 0,
                                                      t16=torch.float16)
    a, da = O.mla_attn_jvp(x, dx, pc, cos, sin, 1e-6, ref_attn)
    h1, dh1 = x + a, dx + da
    m, dm = O.mlp_jvp(h1, dh1, pc, 1e-6)
    _check(y, h1 + m, "block out")
    _check(dy, dh1 + dm, "block tangent")
