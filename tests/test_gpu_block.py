"""GPU parity of the DiT block's fused training kernels against the eager
expression of the reference (models/imf_dit_video.py:136-171): SituAndMul
forward and backward, 16-bit and fp32 I/O, with and without the linear_beta
soft clamp, on 16-byte (F = 2048, 96) and one-element (F = 1365) paths and on
[gate | up] views of one tensor.  The eager form is evaluated in float64 on the
CPU from the same inputs; tolerance: two units in the last place of a 16-bit
I/O dtype (the kernels round once, from fp32), and 2^-16 relative for fp32 I/O,
whose evaluation chain (hardware exp and tanh, then products) carries a few tens
of fp32 ulps (3.7e-6 measured)."""
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

ULP = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -17}


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def situ_eager(g, u, beta, lb):
    act = beta * torch.tanh(g / beta) * torch.sigmoid(g)
    if lb is not None:
        u = lb * torch.tanh(u / lb)
    return act * u


def close(a, b, dt):
    """Per element within 2 ulp of the I/O dtype, plus an absolute floor of
    2 ulp of the tensor's largest magnitude for fp32 I/O: in the saturated clamp
    1 - tanh^2 cancels in fp32 (as in eager torch's tanh_backward), leaving
    elements ~1e-7 of the largest one without relative accuracy."""
    a, b = a.double().cpu(), b.double().cpu()
    floor = 1.0 if dt == torch.float32 else 1e-3
    tol = 2 * ULP[dt] * b.abs() + 2 * ULP[dt] * b.abs().max() * floor + 1e-30
    return bool(((a - b).abs() <= tol).all()), float(((a - b).abs() / (b.abs() + 1e-30)).max())


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("F", [2048, 1365, 96])
@pytest.mark.parametrize("lb", [25.0, None])
@pytest.mark.parametrize("split", [False, True])
def test_situ_mul_forward_backward(dt, F, lb, split):
    from imfvideo_amd.imf_dit_video import SituAndMul
    say("situ_mul", dt, F, lb, split)
    g = torch.Generator().manual_seed(F + (7 if lb else 0) + (3 if split else 0))
    rows = 1000
    beta = 4.0
    scale = 6.0 if lb is None else 40.0   # reach tanh saturation of both branches
    x = (torch.randn(2, rows // 2, 2 * F, generator=g) * scale).to(dt)
    dh = torch.randn(2, rows // 2, F, generator=g).to(dt)
    m = SituAndMul(beta=beta, linear_beta=lb)
    xg = x.cuda().requires_grad_(True)
    if split:
        h = m(xg)                                   # gate / up as views of x
    else:
        gate = xg[..., :F].contiguous()
        up = xg[..., F:].contiguous()
        h = m(gate, up)
    assert h.dtype == dt and h.shape == (2, rows // 2, F)
    h.backward(dh.cuda())
    torch.cuda.synchronize()
    x64 = x.double().requires_grad_(True)
    want = situ_eager(x64[..., :F], x64[..., F:], beta, lb)
    want.backward(dh.double())
    ok, err = close(h.detach(), want.detach(), dt)
    assert ok, ("forward", err)
    ok, err = close(xg.grad, x64.grad, dt)
    assert ok, ("backward", err)


def test_situ_mul_matches_eager_module_on_cpu():
    """The module's CPU branch (the eager fp32 expression) and the fused GPU
    kernels agree to bf16 rounding on the same bf16 inputs."""
    from imfvideo_amd.imf_dit_video import SituAndMul
    say("situ_mul cpu eager vs gpu fused")
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(64, 2 * 512, generator=g) * 5).to(torch.bfloat16)
    m = SituAndMul(beta=4.0, linear_beta=25.0)
    a = m(x).float()
    b = m(x.cuda()).float().cpu()
    assert (a - b).abs().max().item() <= 2 * 2.0 ** -8 * a.abs().max().item()


def _rms_eager(x, w, eps):
    """The module's eager expression (models/imf_dit_video.py:121-133)."""
    xf = x.float()
    normed = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return normed.to(x.dtype) * w


@pytest.mark.parametrize("case", ["f32_512", "bf16_256", "f16_1000", "bf16_heads_view"])
def test_rmsnorm_forward_backward(case):
    """Fused RMSNorm forward / backward against the module's eager expression
    on the CPU (fp32 arithmetic, the same rounding points): y and dx within 2
    ulp of their dtype per element (plus 2 ulp of the largest magnitude: the
    mean and rsqrt round in another order), dw within 1e-5 (fp32) / 1e-4
    (16-bit) of its max-norm."""
    from imfvideo_amd.imf_dit_video import RMSNorm
    say("rmsnorm", case)
    g = torch.Generator().manual_seed(len(case))
    dt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[case.split("_")[0]]
    if case == "bf16_heads_view":
        base = (torch.randn(2, 300, 8, 64, generator=g) * 3).to(dt)
        D = 32
        x = base[..., :D]                                  # strided per-head band
    else:
        D = int(case.split("_")[1])
        base = (torch.randn(2, 300, D, generator=g) * 3).to(dt)
        x = base
    m = RMSNorm(D, eps=1e-6)
    with torch.no_grad():
        m.weight.copy_(1 + 0.5 * torch.randn(D, generator=g))
    dy = torch.randn(x.shape, generator=g)
    # eager on the CPU
    xc = x.detach().clone().requires_grad_(True)
    mc = RMSNorm(D, eps=1e-6)
    with torch.no_grad():
        mc.weight.copy_(m.weight)
    yc = _rms_eager(xc, mc.weight, 1e-6)
    yc.backward(dy)
    # fused on the GPU (x as a view of a GPU tensor, like the MLA head bands)
    mg = m.cuda()
    bg = base.cuda().requires_grad_(True)
    xg = bg[..., :D] if case == "bf16_heads_view" else bg
    yg = mg(xg)
    assert yg.dtype == torch.float32 and yg.shape == x.shape
    yg.backward(dy.cuda())
    torch.cuda.synchronize()
    ulp = ULP[dt] if dt != torch.float32 else 2.0 ** -23

    def within(a, b, u):
        a, b = a.double().cpu(), b.double().cpu()
        return bool(((a - b).abs() <= 2 * u * b.abs() + 2 * u * b.abs().max()).all())

    # y carries one rounding to x's dtype and the fp32 product with w
    assert within(yg.detach(), yc.detach(), max(ulp, 2.0 ** -23))
    dxg = bg.grad[..., :D] if case == "bf16_heads_view" else bg.grad
    assert within(dxg, xc.grad, max(ulp, 2.0 ** -20))
    if case == "bf16_heads_view":
        assert not bg.grad[..., D:].any()
    # dw sums round_x(x r) dy over rows: for 16-bit x a rounding of x r that
    # lands one ulp (2^-8 for bf16) away in a few elements (r is summed in
    # another order) moves the sum by ~1e-5 of its max-norm
    dwg, dwc = mg.weight.grad.double().cpu(), mc.weight.grad.double()
    tol = 1e-5 if dt == torch.float32 else 1e-4
    assert ((dwg - dwc).abs().max() / dwc.abs().max()).item() < tol


@pytest.mark.parametrize("dt,n", [(torch.bfloat16, 3), (torch.bfloat16, 2), (torch.float16, 3)])
def test_norm_fanout_under_autocast(dt, n):
    """The block's residual-stream RMSNorm with n linear consumers under
    autocast: the fused forward equals the cast of the module's fp32 output bit
    for bit, and the backward (the consumers' 16-bit gradients summed in fp32,
    plus the residual's gradient of x) matches eager autograd of
    x + norm(x).to(dt) used n times, on the CPU in fp32."""
    from imfvideo_amd.imf_dit_video import RMSNorm, _norm_fanout
    say("norm fan-out", dt, n)
    g = torch.Generator().manual_seed(n + (1 if dt == torch.float16 else 0))
    D = 512
    x = torch.randn(2, 777, D, generator=g) * 2
    w = 1 + 0.5 * torch.randn(D, generator=g)
    dys = [torch.randn(2, 777, D, generator=g).to(dt) for _ in range(n)]
    dpass = torch.randn(2, 777, D, generator=g)
    m = RMSNorm(D, eps=1e-6).cuda()
    with torch.no_grad():
        m.weight.copy_(w)
    xg = x.cuda().requires_grad_(True)
    with torch.autocast("cuda", dtype=dt):
        outs = _norm_fanout(xg, m, n)
    xp, ys = outs[0], outs[1:]
    assert len(ys) == n and all(y.dtype == dt for y in ys)
    want = _rms_eager(x, w, 1e-6).to(dt)
    assert torch.equal(ys[0].cpu(), want) or (ys[0].cpu().float() - want.float()).abs().max() <= \
        ULP[dt] * want.float().abs().max()
    torch.autograd.backward([xp] + list(ys), [dpass.cuda()] + [d.cuda() for d in dys])
    torch.cuda.synchronize()
    xc = x.clone().requires_grad_(True)
    wc = w.clone().requires_grad_(True)
    yc = _rms_eager(xc, wc, 1e-6)
    (xc * 1.0).backward(dpass, retain_graph=True)
    yc.backward(sum(d.float() for d in dys))
    ok = ((xg.grad.cpu() - xc.grad).abs() <= 1e-5 * xc.grad.abs() + 1e-5 * xc.grad.abs().max()).all()
    print(f"  dx max rel {((xg.grad.cpu() - xc.grad).abs().max() / xc.grad.abs().max()).item():.2e}",
          flush=True)
    assert ok
    dwg = m.weight.grad.cpu()
    assert ((dwg - wc.grad).abs().max() / wc.grad.abs().max()).item() < 1e-5


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_gate_mul_matches_torch(dt):
    """The fused output gate a * sigmoid(g) against torch's own elementwise
    kernels on the same 16-bit GPU tensors (sigmoid, mul and their backward):
    forward and both gradients within one unit in the last place (the
    exponential's implementation may differ by an fp32 ulp)."""
    from imfvideo_amd.imf_dit_video import _GateMulFunction
    say("gate mul", dt)
    g = torch.Generator().manual_seed(4)
    a = (torch.randn(2, 999, 512, generator=g) * 3).to(dt).cuda()
    gt = (torch.randn(2, 999, 512, generator=g) * 4).to(dt).cuda()
    dout = torch.randn(2, 999, 512, generator=g).to(dt).cuda()
    a1, g1 = a.clone().requires_grad_(True), gt.clone().requires_grad_(True)
    o1 = _GateMulFunction.apply(a1, g1)
    o1.backward(dout)
    a2, g2 = a.clone().requires_grad_(True), gt.clone().requires_grad_(True)
    o2 = a2 * torch.sigmoid(g2)
    o2.backward(dout)
    torch.cuda.synchronize()
    for got, want in ((o1, o2), (a1.grad, a2.grad), (g1.grad, g2.grad)):
        got, want = got.detach().float().cpu(), want.detach().float().cpu()
        bad = (got - want).abs() > ULP[dt] * want.abs() + 1e-30
        print(f"  differ {bad.float().mean().item():.2e}", flush=True)
        assert not bad.any()


def test_block_forward_backward_fanout_matches_plain_norms():
    """A TransformerBlock under bf16 autocast with the fused norm fan-out and
    the same block with the fan-out switched off (norm(x) then the consumers'
    own casts) agree: outputs bit for bit, gradients to fp32 summation order."""
    from functools import partial
    import imfvideo_amd.imf_dit_video as M
    from imfvideo_amd.sla2_cube_qat import SLA2CubeQATAttentionImpl
    say("block with / without the norm fan-out")
    torch.manual_seed(0)
    impl = partial(SLA2CubeQATAttentionImpl, seq_len=640, num_heads=8, grid=(4, 8, 20),
                   tile=(4, 4, 4), topk=0.5, pre_permuted=True)
    blk = M.TransformerBlock(512, 8, 256, 128, 32, 32, 64, mlp_ratio=4,
                             weight_init_constant=0.5, attn_impl=impl).cuda()
    with torch.no_grad():
        blk.attn_scale.fill_(0.1)
        blk.mlp_scale.fill_(0.1)
    g = torch.Generator().manual_seed(1)
    L = 640
    x = torch.randn(2, L, 512, generator=g).cuda()
    cos, sin = (t.cuda() for t in M.precompute_axial_rope_3d(32, (4, 8, 20), 0,
                                                             axis_dims=(8, 12, 12)))
    dy = torch.randn(2, L, 512, generator=g).cuda()

    def run(fanout):
        saved = M._norm_fanout
        if not fanout:
            M._norm_fanout = lambda x, norm, n: (x,) + (norm(x),) * n
        try:
            blk.zero_grad(set_to_none=True)
            xg = x.clone().requires_grad_(True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                out = blk(xg, cos, sin)
            out.backward(dy)
            torch.cuda.synchronize()
            return out.detach(), xg.grad, {k: p.grad.clone() for k, p in blk.named_parameters()
                                           if p.grad is not None}
        finally:
            M._norm_fanout = saved

    o1, dx1, g1 = run(True)
    o0, dx0, g0 = run(False)
    assert torch.equal(o1, o0)
    rel = lambda a, b: ((a - b).norm() / b.norm().clamp_min(1e-30)).item()
    print(f"  dx rel {rel(dx1, dx0):.2e}", flush=True)
    assert rel(dx1, dx0) < 1e-5
    assert g1.keys() == g0.keys() and len(g0) > 10
    for k in g0:
        assert rel(g1[k], g0[k]) < 1e-4, k


def _rope_eager(x, c, s):
    """apply_rotary_pos_emb's eager expression (models/imf_dit_video.py:266-284)."""
    xf = x.float()
    re, im = xf[..., 0::2], xf[..., 1::2]
    c, s = c[None, :, None, :], s[None, :, None, :]
    return torch.stack([re * c - im * s, re * s + im * c], dim=-1).flatten(-2).to(x.dtype)


@pytest.mark.parametrize("case", ["bf16_heads", "bf16_shared_key", "f16_heads", "f32_heads"])
def test_rope_forward_backward(case):
    """RoPE forward and backward (the inverse rotation of the gradient) on
    strided views as the MLA sublayer passes them, against the eager expression
    on the CPU: within 2 ulp of the dtype per element, plus 2 ulp of the largest
    magnitude (the cosine / sine products round in another order)."""
    from imfvideo_amd.imf_dit_video import apply_rotary_pos_emb, precompute_axial_rope_3d
    say("rope", case)
    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[case.split("_")[0]]
    g = torch.Generator().manual_seed(len(case))
    cos, sin = precompute_axial_rope_3d(32, (3, 8, 8), 0, axis_dims=(8, 12, 12))
    L = cos.shape[0]
    if case == "bf16_shared_key":
        base = (torch.randn(2, L, 128 + 32, generator=g) * 2).to(dt)
        view = lambda t: t[..., 128:].unsqueeze(2)            # (b, l, 1, dr)
    else:
        base = (torch.randn(2, L, 4, 64, generator=g) * 2).to(dt)
        view = lambda t: t[..., 32:]                          # (b, l, H, dr) band
    dout = torch.randn(view(base).shape, generator=g)
    xc = base.clone().requires_grad_(True)
    yc = _rope_eager(view(xc), cos, sin)
    yc.backward(dout.to(dt))
    xg = base.cuda().requires_grad_(True)
    yg = apply_rotary_pos_emb(view(xg), cos.cuda(), sin.cuda())
    assert yg.dtype == dt and yg.shape == yc.shape
    yg.backward(dout.to(dt).cuda())
    torch.cuda.synchronize()
    u = ULP[dt] if dt != torch.float32 else 2.0 ** -22

    def within(a, b):
        a, b = a.double().cpu(), b.double().cpu()
        return bool(((a - b).abs() <= 2 * u * b.abs() + 2 * u * b.abs().max()).all())

    assert within(yg.detach(), yc.detach())
    assert within(xg.grad, xc.grad)


@pytest.mark.parametrize("dim", [512, 100])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_residual_scale_forward_backward(dt, dim):
    """x + a * scale (the block's ReZero residual): forward and da bit-identical
    to the eager expression on the CPU (product and sum rounded separately);
    the scale gradient, a sum over rows in another order, within 1e-6.  A
    width of 512 takes the 16-byte-access forward, 100 the per-element one."""
    from imfvideo_amd.imf_dit_video import _residual
    say("residual scale", dt, dim)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, 333, dim, generator=g)
    a = torch.randn(2, 333, dim, generator=g).to(dt)
    s = (0.1 * torch.randn(dim, generator=g))
    dy = torch.randn(2, 333, dim, generator=g)
    xc, ac, sc = (t.clone().requires_grad_(True) for t in (x, a, s))
    yc = xc + ac * sc
    yc.backward(dy)
    xg, ag, sg = (t.cuda().requires_grad_(True) for t in (x, a, s))
    yg = _residual(xg, ag, sg)
    yg.backward(dy.cuda())
    torch.cuda.synchronize()
    assert torch.equal(yg.detach().cpu(), yc.detach())
    assert torch.equal(xg.grad.cpu(), xc.grad)
    assert torch.equal(ag.grad.cpu(), ac.grad)
    assert ((sg.grad.cpu() - sc.grad).abs().max() / sc.grad.abs().max()).item() < 1e-6


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_attn_operands_and_gate_match_torch(dt):
    """The fused operand layout (cat of the halves, the shared key band expanded
    over the heads, permute, .half()) and the fused output gate (permute,
    .to(float32), fp32 gate, the projection's autocast cast) against torch's own
    ops on the same GPU tensors: operands and their gradients bit for bit; the
    gate's output and gradients within one unit in the last place (the
    sigmoid's exponential may differ by an fp32 ulp)."""
    from imfvideo_amd.imf_dit_video import _AttnGateFunction, _AttnInFunction
    say("attention operands and gate", dt)
    g = torch.Generator().manual_seed(7)
    B, L, H = 2, 333, 8
    qn = torch.randn(B, L, H, 32, generator=g).cuda()            # fp32 norm output
    qr = torch.randn(B, L, H, 32, generator=g).to(dt).cuda()
    kn = torch.randn(B, L, H, 32, generator=g).cuda()
    kr = torch.randn(B, L, 1, 32, generator=g).to(dt).cuda()
    kv = torch.randn(B, L, H, 96, generator=g).to(dt).cuda()
    dq, dk, dv = (torch.randn(B, H, L, 64, generator=g).half().cuda() for _ in range(3))
    leaves = lambda: [t.clone().requires_grad_(True) for t in (qn, qr, kn, kr, kv)]

    a = leaves()
    qh, kh, vh = _AttnInFunction.apply(a[0], a[1], a[2], a[3], a[4][..., 32:])
    torch.autograd.backward((qh, kh, vh), (dq, dk, dv))
    b = leaves()
    q = torch.cat([b[0], b[1]], -1)
    k = torch.cat([b[2], b[3].expand(B, L, H, 32)], -1)
    tm = lambda x: x.permute(0, 2, 1, 3).half().contiguous()
    qe, ke, ve = tm(q), tm(k), tm(b[4][..., 32:])
    torch.autograd.backward((qe, ke, ve), (dq, dk, dv))
    torch.cuda.synchronize()
    for got, want in ((qh, qe), (kh, ke), (vh, ve)):
        assert torch.equal(got, want)
    for i, (x, y) in enumerate(zip(a, b)):
        assert x.grad.dtype == y.grad.dtype and torch.equal(x.grad, y.grad), i

    o = (torch.randn(B, H, L, 64, generator=g) * 2).half().cuda()
    gl = (torch.randn(B, L, H * 64, generator=g) * 3).to(dt).cuda()
    dy = torch.randn(B, L, H * 64, generator=g).to(dt).cuda()
    o1, g1 = o.clone().requires_grad_(True), gl.clone().requires_grad_(True)
    y1 = _AttnGateFunction.apply(o1, g1)
    y1.backward(dy)
    o2, g2 = o.clone().requires_grad_(True), gl.clone().requires_grad_(True)
    y2 = (o2.permute(0, 2, 1, 3).to(torch.float32).reshape(B, L, H * 64)
          * torch.sigmoid(g2)).to(dt)
    y2.backward(dy)
    torch.cuda.synchronize()
    assert y1.dtype == dt and o1.grad.dtype == torch.float16 and g1.grad.dtype == dt
    for got, want, u in ((y1, y2, ULP[dt]), (o1.grad, o2.grad, ULP[torch.float16]),
                         (g1.grad, g2.grad, ULP[dt])):
        got, want = got.detach().float().cpu(), want.detach().float().cpu()
        bad = (got - want).abs() > u * want.abs() + 1e-30
        print(f"  differ {bad.float().mean().item():.2e}", flush=True)
        assert not bad.any()


def test_block_fused_attention_path_matches_eager_layout():
    """A TransformerBlock under bf16 autocast with the fused attention operand /
    gate path and the same block on the eager cat / permute / gate path: outputs
    within one bf16 ulp and gradients to fp32 summation order."""
    from functools import partial
    import imfvideo_amd.imf_dit_video as M
    from imfvideo_amd.sla2_cube_qat import SLA2CubeQATAttentionImpl
    say("block with / without the fused attention operands")
    torch.manual_seed(0)
    impl = partial(SLA2CubeQATAttentionImpl, seq_len=640, num_heads=8, grid=(4, 8, 20),
                   tile=(4, 4, 4), topk=0.5, pre_permuted=True)
    blk = M.TransformerBlock(512, 8, 256, 128, 32, 32, 64, mlp_ratio=4,
                             weight_init_constant=0.5, attn_impl=impl).cuda()
    with torch.no_grad():
        blk.attn_scale.fill_(0.1)
        blk.mlp_scale.fill_(0.1)
    g = torch.Generator().manual_seed(2)
    L = 640
    x = torch.randn(2, L, 512, generator=g).cuda()
    cos, sin = (t.cuda() for t in M.precompute_axial_rope_3d(32, (4, 8, 20), 0,
                                                             axis_dims=(8, 12, 12)))
    dy = torch.randn(2, L, 512, generator=g).cuda()

    def run(fused):
        saved = M._tile_major_operands_ok
        if not fused:
            M._tile_major_operands_ok = lambda *a: False
        try:
            blk.zero_grad(set_to_none=True)
            xg = x.clone().requires_grad_(True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                out = blk(xg, cos, sin)
            out.backward(dy)
            torch.cuda.synchronize()
            return out.detach(), xg.grad, {k: p.grad.clone() for k, p in blk.named_parameters()
                                           if p.grad is not None}
        finally:
            M._tile_major_operands_ok = saved

    o1, dx1, g1 = run(True)
    o0, dx0, g0 = run(False)
    rel = lambda a, b: ((a - b).norm() / b.norm().clamp_min(1e-30)).item()
    print(f"  out max {(o1 - o0).abs().max().item():.2e} dx rel {rel(dx1, dx0):.2e}", flush=True)
    assert ((o1 - o0).abs() <= 2.0 ** -7 * o0.abs() + 1e-6).all()
    assert rel(dx1, dx0) < 1e-4
    assert g1.keys() == g0.keys() and len(g0) > 10
    for k in g0:
        assert rel(g1[k], g0[k]) < 1e-3, k
