"""GPU runs of the reference's own test recipes and of the API paths its callers
use (marked gpu).

* tests/test_sla2_cube_qat.py:34-45 replayed: the INT8 cube JVP against
  torch.func.jvp of the unquantised dense fp32 form (mvs_dense_ref) on the same
  LUT, rel-Frobenius o < 3e-2 and do < 8e-2 (the reference's bound).
* tests/test_sla2_cube_qat.py:47-67 replayed: the module with use_int8 True and
  False, forward and backward finite, alpha gradient non-zero, the two
  forwards within rel 5e-2; plus the 16-bit module path against the oracle.
* tests/test_mla_video_sparse_jvp.py replayed for E = 64 (this build's tile):
  the 16-bit cube JVP against torch.func.jvp of mvs_dense_ref with
  non-identity router projections, the reference's fp16 bound 2e-2 / 5e-2.
* Tile-major residency (models/imf_dit_video.py:786-800, 1014-1018): the
  module with pre_permuted=True and the MLA sublayer JVP with
  cube["pre_permuted"] on tile-ordered tokens and permuted RoPE tables equal
  the model-order runs, and the oracle.
"""
import pytest
import torch

from oracle import sla2_oracle as O
from tests.helpers import max_abs, rel_l2
from tests.test_gpu_parity import TOL_MAX, TOL_REL, cuda, say

pytestmark = pytest.mark.gpu


def rel_fro(a, b):
    return rel_l2(a.detach().cpu(), b.detach().cpu())


def ref_geometry(seed, B=2, H=2, Np=4, P=18, scale_tan=1.0):
    """The reference tests' shapes (D = 64, E = 64, ragged prefix of P tokens)
    drawn from a CPU generator: q..dv N(0,1) fp32, alpha U(0.1, 0.9) (H, Mb)."""
    g = torch.Generator().manual_seed(seed)
    L = Np * 64 + P
    x = [torch.randn(B, H, L, 64, generator=g) for _ in range(3)]
    x += [torch.randn(B, H, L, 64, generator=g) * scale_tan for _ in range(3)]
    alpha = torch.rand(H, Np + -(-P // 64), generator=g) * 0.8 + 0.1
    return x, alpha, Np, P, g


def dense_jvp(x, alpha, lut, Np, P, dtype=torch.float64):
    """torch.func.jvp of mvs_dense_ref on the CPU (float64 by default)."""
    from imfvideo_amd.mla_video_sparse_jvp import mvs_dense_ref
    q, k, v, dq, dk, dv = (t.to(dtype) for t in x)
    lut = torch.as_tensor(lut).cpu()
    a = alpha.to(dtype)
    return torch.func.jvp(lambda a_, b_, c_: mvs_dense_ref(a_, b_, c_, a, lut, Np, 64, P),
                          (q, k, v), (dq, dk, dv))


def test_reference_recipe_int8_jvp_against_the_dense_jvp():
    say("tests/test_sla2_cube_qat.py:34-45 on the GPU")
    from imfvideo_amd.mla_video_sparse_jvp import route_tiles
    from imfvideo_amd.sla2_cube_qat import sla2_cube_qat_jvp, sla2_cube_qat_jvp_fused
    x, alpha, Np, P, _ = ref_geometry(0)
    q, k, v, dq, dk, dv = (cuda(t) for t in x)
    lut, T = route_tiles(q, k, 0.5, Np, 64, P)
    assert T == 2 and lut.shape == (2, 2, 5, 2)
    o_ref, do_ref = dense_jvp(x, alpha, lut, Np, P)
    for fn in (sla2_cube_qat_jvp, sla2_cube_qat_jvp_fused):
        o, do = fn(q, k, v, dq, dk, dv, cuda(alpha), 0.5, Np, 64, P, lut=lut, T=T)
        torch.cuda.synchronize()
        r_o, r_do = rel_fro(o, o_ref), rel_fro(do, do_ref)
        print(f"  {fn.__name__}: o {r_o:.2e} do {r_do:.2e} (reference records 9.7e-3 / 1.1e-2)",
              flush=True)
        assert o.dtype == torch.float32 and do.dtype == torch.float32
        assert r_o < 3e-2 and r_do < 8e-2


def _module(int8, pre_permuted=False, seed=1):
    from imfvideo_amd.sla2_cube_qat import SLA2CubeQATAttentionImpl
    torch.manual_seed(seed)
    return SLA2CubeQATAttentionImpl(head_dim=64, seq_len=274, num_heads=2, grid=(4, 8, 8),
                                    tile=(4, 4, 4), topk=0.5, alpha_init=0.9, use_int8=int8,
                                    pre_permuted=pre_permuted).cuda()


def test_reference_recipe_module_int8_and_16bit():
    say("tests/test_sla2_cube_qat.py:47-67 on the GPU")
    outs = {}
    for int8 in (True, False):
        mod = _module(int8)
        g = torch.Generator().manual_seed(21)
        x = cuda(torch.randn(2, 274, 2, 64, generator=g)).requires_grad_()
        o_m = mod(x, x * 0.9, x * 1.1)
        assert o_m.shape == x.shape and o_m.dtype == x.dtype and torch.isfinite(o_m).all()
        o_m.square().mean().backward()
        ga = mod.alpha_logit.grad
        assert ga is not None and torch.isfinite(ga).all() and ga.abs().sum() > 0
        assert torch.isfinite(x.grad).all()
        outs[int8] = o_m.detach()
    rel = rel_fro(outs[True], outs[False])
    print(f"  int8 vs 16-bit forward rel {rel:.2e}", flush=True)
    assert rel < 5e-2


def test_module_16bit_path_matches_the_oracle():
    """use_int8=False: the 16-bit sparse training forward (S = q.k^T on 16-bit
    MFMA, O += round16(P) V, the prefix tail attended through lut_aug), the
    training forward's linear branch and mix, and the straight-through
    backward, against the oracle's int8=False restatement; the no-grad
    (guidance) forward equals the autograd one."""
    say("SLA2CubeQATAttentionImpl(use_int8=False) forward + backward vs oracle")
    mod = _module(False)
    with torch.no_grad():
        mod.alpha_logit.add_(torch.linspace(-1, 1, mod.alpha_logit.numel(),
                                            device="cuda").view_as(mod.alpha_logit))
    g = torch.Generator().manual_seed(23)
    x = [torch.randn(2, 274, 2, 64, generator=g) for _ in range(4)]
    with torch.no_grad():
        out_ng = mod(*(cuda(t) for t in x[:3])).cpu()
    xs = [cuda(t).requires_grad_() for t in x[:3]]
    out = mod(*xs)
    (out * cuda(x[3])).sum().backward()
    assert torch.equal(out.detach().cpu(), out_ng)
    perm, inv = mod.perm.cpu(), mod.inv.cpu()
    tm = lambda t: t.permute(0, 2, 1, 3)[:, :, perm].half().float()
    qh, kh, vh, doh = (tm(t) for t in x)
    lut, T, _, _ = O.route(qh, kh, 0.5, mod.Np, mod.prefix_len, torch.eye(64), torch.eye(64))
    a = torch.sigmoid(mod.alpha_logit.detach().cpu())
    fwd = O.train_fwd(qh, kh, vh, a, lut, mod.Np, mod.prefix_len, t16=torch.float16, int8=False)
    back = lambda t: t[:, :, inv].permute(0, 2, 1, 3)
    eo = back(fwd["o"])
    print(f"  o max {max_abs(out_ng, eo):.2e} rel {rel_l2(out_ng, eo):.2e}", flush=True)
    assert max_abs(out_ng, eo) < TOL_MAX and rel_l2(out_ng, eo) < TOL_REL
    assert torch.allclose(mod.logit_max_log2.cpu(), fwd["lse"].amax(dim=(0, 2)), atol=1e-3)
    ref = O.train_bwd(qh, kh, vh, a, lut, mod.Np, mod.prefix_len, fwd, doh, t16=torch.float16)
    for t_, name in zip(xs, ("dq", "dk", "dv")):
        got, want = t_.grad.cpu(), back(ref[name])
        print(f"  {name} max {max_abs(got, want):.2e} rel {rel_l2(got, want):.2e}", flush=True)
        assert rel_l2(got, want) < TOL_REL and max_abs(got, want) < TOL_MAX * max(1, want.abs().max())
    assert rel_l2(mod.alpha_logit.grad.cpu(), ref["d_alpha"]) < 1e-3


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_reference_recipe_mla_video_sparse_jvp(dt):
    """tests/test_mla_video_sparse_jvp.py with E = 64: grid (8, 8, 8), tile
    (4, 4, 4) -> Np = 8, P = 18, router projections eye + 0.05 randn, top-k
    0.25 -> T = 2, block_m = 32.  Against torch.func.jvp of mvs_dense_ref (fp64)
    at the reference's fp16 bound; fp32 inputs are computed at fp16 here, so
    they take that bound too.  Then against the dense form of the inputs
    rounded to the compute type, where only the 16-bit P / T operands and the
    summation order remain."""
    say("tests/test_mla_video_sparse_jvp.py (E = 64) on the GPU,", dt)
    from imfvideo_amd.mla_video_sparse_jvp import mla_video_sparse_jvp, route_tiles
    x, alpha, Np, P, g = ref_geometry(3, Np=8)
    proj_q = torch.eye(64) + 0.05 * torch.randn(64, 64, generator=g)
    proj_k = torch.eye(64) + 0.05 * torch.randn(64, 64, generator=g)
    ct = torch.float16 if dt == torch.float32 else dt   # the compute type
    # routed on the inputs as given (fp32 unrounded), as lut=None does below
    lut, T = route_tiles(*(cuda(t.to(dt)) for t in x[:2]), 0.25, Np, 64, P,
                         proj_q=cuda(proj_q), proj_k=cuda(proj_k))
    assert T == 2
    o_ref, do_ref = dense_jvp(x, alpha, lut, Np, P)
    gx = [cuda(t.to(dt)) for t in x]
    o, do = mla_video_sparse_jvp(*gx, cuda(alpha), 0.25, Np, 64, P, lut=lut, T=T, block_m=32)
    torch.cuda.synchronize()
    r_o, r_do = rel_fro(o, o_ref), rel_fro(do, do_ref)
    print(f"  vs fp32 inputs: o {r_o:.2e} do {r_do:.2e}", flush=True)
    assert o.dtype == torch.float32 and r_o < 2e-2 and r_do < 5e-2
    o_r, do_r = dense_jvp([t.to(ct) for t in x], alpha, lut, Np, P)
    r_o, r_do = rel_fro(o, o_r), rel_fro(do, do_r)
    print(f"  vs rounded inputs: o {r_o:.2e} do {r_do:.2e}", flush=True)
    assert r_o < 5e-3 and r_do < 1e-2
    # lut=None routes with route_tiles on the rounded inputs: the same selection here
    o2, do2 = mla_video_sparse_jvp(*gx, cuda(alpha), 0.25, Np, 64, P, proj_q=cuda(proj_q),
                                   proj_k=cuda(proj_k))
    assert torch.equal(o2, o) and torch.equal(do2, do)


@pytest.mark.xfail(strict=True, reason="fp32 inputs are computed in fp16 on the 16-bit MFMA path "
                   "(documented deviation): o ~1e-2 against the reference's fp32 bound 2e-4")
def test_reference_fp32_bound_of_the_non_qat_cube_jvp():
    """The reference's fp32 tolerance (tests/test_mla_video_sparse_jvp.py:54: o 2e-4,
    do 2e-3 against the dense fp32 JVP).  Its fp32 mode runs IEEE fp32 dots; this
    build's kernels take 16-bit operands, so fp32 inputs get the fp16 bound
    (checked above) and this bound is not met: strict xfail, so a future fp32
    path that meets it turns the test into a failure to remove the marker."""
    from imfvideo_amd.mla_video_sparse_jvp import mla_video_sparse_jvp, route_tiles
    x, alpha, Np, P, g = ref_geometry(3, Np=8)
    proj_q = torch.eye(64) + 0.05 * torch.randn(64, 64, generator=g)
    proj_k = torch.eye(64) + 0.05 * torch.randn(64, 64, generator=g)
    lut, T = route_tiles(*(cuda(t) for t in x[:2]), 0.25, Np, 64, P,
                         proj_q=cuda(proj_q), proj_k=cuda(proj_k))
    o_ref, do_ref = dense_jvp(x, alpha, lut, Np, P)
    o, do = mla_video_sparse_jvp(*(cuda(t) for t in x), cuda(alpha), 0.25, Np, 64, P, lut=lut,
                                 T=T, block_m=32)
    torch.cuda.synchronize()
    r_o, r_do = rel_fro(o, o_ref), rel_fro(do, do_ref)
    print(f"  fp32 inputs: o {r_o:.2e} (reference bound 2e-4) do {r_do:.2e} (2e-3)", flush=True)
    assert r_o < 2e-4 and r_do < 2e-3


def test_module_pre_permuted_matches_model_order():
    """pre_permuted=True on tile-ordered tokens (the model keeps the sequence
    tile-major) gives the model-order module's result at the tile positions,
    bit for bit, forward and backward (and therefore the oracle's, which the
    model-order module is checked against)."""
    say("SLA2CubeQATAttentionImpl(pre_permuted=True) vs model order")
    a_mod, b_mod = _module(True), _module(True, pre_permuted=True)
    with torch.no_grad():
        a_mod.alpha_logit.add_(torch.linspace(-1, 1, 10, device="cuda").view(2, 5))
        b_mod.alpha_logit.copy_(a_mod.alpha_logit)
    perm = a_mod.perm
    g = torch.Generator().manual_seed(29)
    x = [cuda(torch.randn(2, 274, 2, 64, generator=g)) for _ in range(4)]
    with torch.no_grad():
        assert torch.equal(a_mod(*x[:3])[:, perm], b_mod(*(t[:, perm] for t in x[:3])))
    xa = [t.clone().requires_grad_() for t in x[:3]]
    xb = [t[:, perm].clone().requires_grad_() for t in x[:3]]
    oa, ob = a_mod(*xa), b_mod(*xb)
    assert torch.equal(oa[:, perm], ob)
    (oa * x[3]).sum().backward()
    (ob * x[3][:, perm]).sum().backward()
    for ta, tb in zip(xa, xb):
        assert torch.equal(ta.grad[:, perm], tb.grad)
    assert torch.equal(a_mod.alpha_logit.grad, b_mod.alpha_logit.grad)
    # and the oracle, directly, on the tile-ordered run
    tm = lambda t: t.permute(0, 2, 1, 3).half().float().cpu()
    qh, kh, vh = (tm(t[:, perm]) for t in x[:3])
    lut, _, _, _ = O.route(qh, kh, 0.5, b_mod.Np, b_mod.prefix_len, torch.eye(64), torch.eye(64))
    a = torch.sigmoid(b_mod.alpha_logit.detach().cpu())
    eo = O.train_fwd(qh, kh, vh, a, lut, b_mod.Np, b_mod.prefix_len, t16=torch.float16)["o"]
    got = ob.detach().cpu().permute(0, 2, 1, 3)
    assert max_abs(got, eo) < TOL_MAX and rel_l2(got, eo) < TOL_REL


def test_sublayer_jvp_pre_permuted_matches_model_order(monkeypatch):
    """The MLA sublayer JVP with cube["pre_permuted"] on tile-ordered tokens and
    RoPE tables permuted once by the caller (models/imf_dit_video.py:786-800)
    equals the model-order run at the tile positions, and the oracle (whose
    attention takes the LUT the GPU routed)."""
    say("attn_sublayer_jvp cube pre_permuted vs model order")
    from imfvideo_amd import ops
    from imfvideo_amd.mla_jvp_fast import attn_sublayer_jvp, mla_fp16_cache
    from imfvideo_amd.mla_video_sparse_jvp import tile_permutation
    from tests.block_ref import LutRecorder
    from tests.test_gpu_mla import gpu_params, params, rope
    p, g = params(31)
    B, P = 2, 18
    S = 256 + P
    h = torch.randn(B, S, 256, generator=g)
    dh = 0.1 * torch.randn(B, S, 256, generator=g)
    cos, sin = rope(S, P)
    perm, inv, Np = tile_permutation((4, 8, 8), (4, 4, 4), P, torch.device("cpu"))
    alpha = torch.rand(2, 5, generator=g) * 0.8 + 0.1
    pg = gpu_params(p)
    w16 = mla_fp16_cache(pg)
    cube = {"alpha": cuda(alpha), "topk": 0.5, "Np": Np, "E": 64, "P": P, "perm": perm,
            "inv": inv}
    rec = LutRecorder(ops.route_topk)
    monkeypatch.setattr(ops, "route_topk", rec)
    pg["cube"] = dict(cube, pre_permuted=False)
    a1, da1 = attn_sublayer_jvp(cuda(h), cuda(dh), pg, w16, cuda(cos), cuda(sin), 1e-6)
    pg["cube"] = dict(cube, pre_permuted=True)
    a2, da2 = attn_sublayer_jvp(cuda(h[:, perm]), cuda(dh[:, perm]), pg, w16,
                                cuda(cos[perm]), cuda(sin[perm]), 1e-6)
    torch.cuda.synchronize()
    assert len(rec.luts) == 2 and torch.equal(rec.luts[0], rec.luts[1])
    for u, w_, n in ((a1[:, perm], a2, "a"), (da1[:, perm], da2, "da")):
        r = rel_fro(u, w_)
        print(f"  {n}: model order vs tile order rel {r:.2e}", flush=True)
        assert r < 1e-5
    lut = rec.luts[1].numpy()
    ref_attn = lambda q, k, v, dq, dk, dv: O.cube_jvp(q, k, v, dq, dk, dv, alpha, lut, Np, P,
                                                      t16=torch.float16)
    want = O.mla_attn_jvp(h[:, perm], dh[:, perm], p, cos[perm], sin[perm], 1e-6, ref_attn)
    for got, w_, n in ((a2, want[0], "a"), (da2, want[1], "da")):
        got, w_ = got.cpu().double(), w_.double()
        bound = TOL_MAX * max(1.0, w_.abs().max().item())
        print(f"  {n} vs oracle: max {max_abs(got, w_):.2e} rel {rel_l2(got, w_):.2e}",
              flush=True)
        assert max_abs(got, w_) < bound and rel_l2(got, w_) < TOL_REL
