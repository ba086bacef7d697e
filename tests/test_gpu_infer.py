"""GPU parity of the 1-D SLA2 inference path (SLA2.forward without gradients)
against the CPU oracle (marked gpu).

INT8 tensors and scales bit for bit (round-half-away law, any block size, V in
the MFMA fragment order); the sparse branch, the 16-bit block states and the
mixed output within the north-star tolerance (max-abs 2e-2, rel-L2 1e-2) and
tighter where the kernels follow the oracle operation by operation.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import sla2_oracle as O
from tests.helpers import max_abs, rel_l2

pytestmark = pytest.mark.gpu
TOL_MAX, TOL_REL = 2e-2, 1e-2


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def cuda(t):
    return t.to("cuda")


def _inputs(seed, B, H, L, dt):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(B, H, L, 64, generator=g).to(dt) for _ in range(3)]


@pytest.mark.parametrize("E", [32, 128, 256])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_quantize_other_block_sizes(E, dt):
    from imfvideo_amd import ops
    say("quantize E", E, dt)
    x = _inputs(60 + E, 1, 3, 583, dt)[0] * 2.5
    x8, xs = ops.quantize(cuda(x.to(dt)), E)
    want_q, want_s = O.quantize_blocks(x.to(dt).float(), E)
    assert np.array_equal(x8.cpu().numpy(), want_q)
    assert np.array_equal(xs.cpu().numpy(), want_s)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_quantize_v8f_fragment_order(dt):
    from imfvideo_amd import ops
    say("quantize_v8f", dt)
    v = _inputs(70, 1, 2, 583, dt)[2]
    v8f, vs = ops.quantize_v8f(cuda(v))
    want_q, want_s = O.quantize_blocks(v.float())
    assert np.array_equal(vs.cpu().numpy(), want_s)
    nb = -(-583 // 64)
    w = np.zeros((1, 2, nb * 64, 64), np.int8)
    w[:, :, :583] = want_q
    # byte s of lane (g, rr) of column tile ct = V8[16 (s >> 2) + 4 g + (s & 3)][16 ct + rr]:
    # tile rows (kb, g, i), columns (ct, rr) -> [ct][g][rr][kb][i]
    frag = w.reshape(1, 2, nb, 4, 4, 4, 4, 16).transpose(0, 1, 2, 6, 4, 7, 3, 5)
    assert np.array_equal(v8f.cpu().numpy(), np.ascontiguousarray(frag).reshape(1, 2, nb, 4096))


@pytest.mark.parametrize("bq,qblock", [(64, 64), (64, 32), (128, 128), (128, 64), (256, 128)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_sparse_fwd_int8_matches_oracle(bq, qblock, dt):
    from imfvideo_amd import ops
    say("sparse_fwd_int8 bq", bq, "qblock", qblock, dt)
    L, H = 583, 2
    q, k, v = _inputs(80 + bq + qblock, 1, H, L, dt)
    lut, T = O.route_1d(q.float(), k.float(), 0.3, bq)
    mq = -(-L // bq)
    g = [cuda(t) for t in (q, k, v)]
    q8, qs = ops.quantize(g[0], qblock)
    k8, ks = ops.quantize(g[1])
    v8f, vs = ops.quantize_v8f(g[2])
    o_s, lse, qphi = ops.sparse_fwd_int8(g[0], q8, qs, qblock, k8, ks, v8f, vs,
                                         cuda(torch.as_tensor(lut)), bq)
    torch.cuda.synchronize()
    t16 = dt
    ref = O.infer_1d(q.float(), k.float(), v.float(), torch.ones(H, mq), lut, bq, int8=True,
                     qblock=qblock, t16=t16)
    print(f"  o_s max {max_abs(o_s.cpu(), ref['o_s']):.2e} rel {rel_l2(o_s.cpu(), ref['o_s']):.2e}"
          f"  lse max {max_abs(lse.cpu(), ref['lse']):.2e}", flush=True)
    assert max_abs(o_s.cpu(), ref["o_s"]) < TOL_MAX and rel_l2(o_s.cpu(), ref["o_s"]) < 2e-3
    assert max_abs(lse.cpu(), ref["lse"]) < 1e-4
    assert max_abs(qphi.cpu(), ref["qphi"]) < 2e-3


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_hblocks_states_match_oracle(dt):
    from imfvideo_amd import ops
    say("hblocks_states", dt)
    L, H = 583, 2
    q, k, v = _inputs(90, 1, H, L, dt)
    st = ops.hblocks_states(cuda(k), cuda(v), with_sums=True)
    torch.cuda.synchronize()
    lut, _ = O.route_1d(q.float(), k.float(), 0.3, 128)
    ref = O.infer_1d(q.float(), k.float(), v.float(), torch.ones(H, 5), lut, 128, int8=False,
                     t16=dt)
    hb, zb = st["Hb"].cpu(), st["zb"].cpu()
    # every value is a 16-bit number; phi may differ from torch's softmax by one 16-bit ulp
    assert torch.equal(hb.to(dt).float(), hb)
    print(f"  Hb rel {rel_l2(hb, ref['hall']):.2e}  zb rel {rel_l2(zb, ref['zall']):.2e}",
          flush=True)
    assert rel_l2(hb, ref["hall"]) < 2e-3 and rel_l2(zb, ref["zall"]) < 1e-4
    assert rel_l2(st["Hall"].cpu(), ref["hall"].sum(2)) < 2e-3


@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("bq", [64, 128])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_sla2_infer_matches_oracle(int8, bq, dt):
    from imfvideo_amd import ops
    say("sla2_infer int8", int8, "bq", bq, dt)
    L, H = 1000, 2
    q, k, v = _inputs(100 + bq, 2, H, L, dt)
    mq = -(-L // bq)
    lut, _ = O.route_1d(q.float(), k.float(), 0.25, bq)
    g = torch.Generator().manual_seed(7)
    alpha = 0.1 + 0.8 * torch.rand(H, mq, generator=g)
    o = ops.sla2_infer(cuda(q), cuda(k), cuda(v), cuda(alpha), cuda(torch.as_tensor(lut)), bq,
                       use_int8=int8)
    torch.cuda.synchronize()
    ref = O.infer_1d(q.float(), k.float(), v.float(), alpha, lut, bq, int8=int8, t16=dt)
    got = o.cpu().float()
    print(f"  o max {max_abs(got, ref['o']):.2e} rel {rel_l2(got, ref['o']):.2e}", flush=True)
    assert max_abs(got, ref["o"]) < TOL_MAX and rel_l2(got, ref["o"]) < TOL_REL


@pytest.mark.parametrize("fused", [False, True])
def test_sla2_module_no_grad_is_the_inference_path(fused):
    """SLA2 (bq = 128, use_int8 = True: the reference's defaults) without
    gradients: routing, Q-scale blocks (bq, or block_m = 64 when fused) and
    alpha (head-averaged when fused) as the reference's core.py:98-128."""
    from imfvideo_amd import ops
    from imfvideo_amd.sla2_vendor.core import SLA2
    say("SLA2 no-grad fused", fused)
    torch.manual_seed(3)
    L, H = 1000, 2
    mod = SLA2(64, topk=0.25, bq=128, use_int8=True, fused=fused).cuda()
    q, k, v = _inputs(110, 1, H, L, torch.float16)
    with torch.no_grad():
        o = mod(cuda(q), cuda(k), cuda(v))
        mod.alpha_logit.add_(torch.linspace(-1, 1, mod.alpha_logit.numel(), device="cuda")
                             .view_as(mod.alpha_logit))
        o = mod(cuda(q), cuda(k), cuda(v)).cpu().float()
    a = torch.sigmoid(mod.alpha_logit.detach().float().cpu())
    if fused:
        a = a.mean(0, keepdim=True).expand(H, -1)
    lut, _ = O.route_1d(q.float(), k.float(), 0.25, 128)
    ref = O.infer_1d(q.float(), k.float(), v.float(), a, lut, 128, int8=True,
                     qblock=64 if fused else 128, t16=torch.float16, fused=fused)
    print(f"  o max {max_abs(o, ref['o']):.2e} rel {rel_l2(o, ref['o']):.2e}", flush=True)
    assert max_abs(o, ref["o"]) < TOL_MAX and rel_l2(o, ref["o"]) < TOL_REL


@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("bq", [64, 128, 256])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_sla2_infer_fused_matches_oracle(int8, bq, dt):
    """The fused Algorithm-2 arithmetic (kernel_fused.py:29-124): Q scales per
    block_m = max(32, bq / 2) rows, o_s in fp32 into the mix, the score-form
    complement against the whole-sequence state, head-shared alpha.  The result
    is nearer to the oracle's fused form than to its unfused one."""
    from imfvideo_amd import ops
    say("sla2_infer_fused int8", int8, "bq", bq, dt)
    L, H = 1000, 2
    q, k, v = _inputs(150 + bq, 2, H, L, dt)
    mq = -(-L // bq)
    lut, _ = O.route_1d(q.float(), k.float(), 0.25, bq)
    g = torch.Generator().manual_seed(11)
    a = (0.1 + 0.8 * torch.rand(mq, generator=g))
    o = ops.sla2_infer_fused(cuda(q), cuda(k), cuda(v), cuda(a), cuda(torch.as_tensor(lut)), bq,
                             use_int8=int8)
    torch.cuda.synchronize()
    qb = max(32, bq // 2) if int8 else None
    kw = dict(int8=int8, qblock=qb, t16=dt)
    ah = a.view(1, -1).expand(H, -1)
    ref = O.infer_1d(q.float(), k.float(), v.float(), ah, lut, bq, fused=True, **kw)
    other = O.infer_1d(q.float(), k.float(), v.float(), ah, lut, bq, **kw)
    got = o.cpu().float()
    near, far = rel_l2(got, ref["o"]), rel_l2(got, other["o"])
    print(f"  o max {max_abs(got, ref['o']):.2e} rel {near:.2e} (unfused form {far:.2e})",
          flush=True)
    assert max_abs(got, ref["o"]) < TOL_MAX and near < TOL_REL
    assert near < far


@pytest.mark.parametrize("L,topk,bq", [(256, 0.01, 128), (640, 0.5, 256), (700, 0.1, 64)])
def test_sla2_infer_fused_edge_shapes(L, topk, bq):
    """T = 1, one ragged block, three batch rows (an empty complement is left
    out: the score form then returns a rounding residual over eps, in the
    reference as here)."""
    from imfvideo_amd import ops
    say("sla2_infer_fused edge L", L, "topk", topk, "bq", bq)
    H = 2
    q, k, v = _inputs(160 + L, 3, H, L, torch.bfloat16)
    mq = -(-L // bq)
    lut, T = O.route_1d(q.float(), k.float(), topk, bq)
    g = torch.Generator().manual_seed(12)
    a = 0.1 + 0.8 * torch.rand(mq, generator=g)
    o = ops.sla2_infer_fused(cuda(q), cuda(k), cuda(v), cuda(a), cuda(torch.as_tensor(lut)), bq)
    torch.cuda.synchronize()
    ref = O.infer_1d(q.float(), k.float(), v.float(), a.view(1, -1).expand(H, -1), lut, bq,
                     int8=True, qblock=max(32, bq // 2), t16=torch.bfloat16, fused=True)
    got = o.cpu().float()
    print(f"  T {T} o max {max_abs(got, ref['o']):.2e} rel {rel_l2(got, ref['o']):.2e}",
          flush=True)
    assert torch.isfinite(got).all()
    assert max_abs(got, ref["o"]) < TOL_MAX and rel_l2(got, ref["o"]) < TOL_REL


# ---------------------------------------------------------------------------
# INT8 training forward of the 1-D SLA2 (bq = 128: the reference's default)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("E", [64, 128, 256])
def test_quantize_trunc_law(E):
    from imfvideo_amd import ops
    say("quantize_trunc E", E)
    x = _inputs(120 + E, 1, 3, 583, torch.bfloat16)[0] * 1.7
    x8, xs = ops.quantize_trunc(cuda(x), E)
    want_q, want_s = O.quantize_blocks_trunc(x.float(), E)
    assert np.array_equal(x8.cpu().numpy(), want_q)
    assert np.array_equal(xs.cpu().numpy(), want_s)


@pytest.mark.parametrize("bq", [128, 256])
def test_sla2_int8_training_forward_and_backward(bq):
    """SLA2(use_int8=True, bq) with gradients: the INT8 sparse branch of
    _attn_fwd_qat (truncating law, Q scales per bq rows) and the STE backward."""
    from imfvideo_amd.sla2_vendor.core import SLA2
    say("SLA2 INT8 training bq", bq)
    torch.manual_seed(4)
    L, H = 583, 2
    mq = -(-L // bq)
    mod = SLA2(64, topk=0.3, bq=bq, use_int8=True).cuda()
    q, k, v = _inputs(130 + bq, 1, H, L, torch.float16)
    with torch.no_grad():
        mod(cuda(q), cuda(k), cuda(v))  # creates alpha
        mod.alpha_logit.add_(torch.linspace(-1, 1, mod.alpha_logit.numel(), device="cuda")
                             .view_as(mod.alpha_logit))
    xs = [cuda(t).requires_grad_() for t in (q, k, v)]
    out = mod(*xs)
    g = torch.Generator().manual_seed(9)
    do = torch.randn(1, H, L, 64, generator=g).half()
    (out.float() * cuda(do).float()).sum().backward()
    grads = [t.grad.cpu() for t in xs] + [mod.alpha_logit.grad.cpu()]
    lut, _ = O.route_1d(q.float(), k.float(), 0.3, bq)
    nb = -(-L // 64)
    a = torch.sigmoid(mod.alpha_logit.detach().cpu())
    fwd = O.train_fwd(q.float(), k.float(), v.float(), a, lut, nb, 0, t16=torch.float16,
                      int8=True, bq=bq)
    o = out.detach().cpu().float()
    print(f"  o max {max_abs(o, fwd['o']):.2e} rel {rel_l2(o, fwd['o']):.2e}", flush=True)
    assert max_abs(o, fwd["o"]) < TOL_MAX and rel_l2(o, fwd["o"]) < TOL_REL
    ref = O.train_bwd(q.float(), k.float(), v.float(), a, lut, nb, 0, fwd, do.float(),
                      t16=torch.float16, bq=bq, variant="1d")
    for got, name in zip(grads[:3], ("dq", "dk", "dv")):
        want = ref[name]
        print(f"  {name} max {max_abs(got, want):.2e} rel {rel_l2(got, want):.2e}", flush=True)
        assert rel_l2(got, want) < TOL_REL and max_abs(got, want) < TOL_MAX * max(1, want.abs().max())
    assert rel_l2(grads[3], ref["d_alpha"]) < 1e-2


@pytest.mark.parametrize("L,topk,bq", [(40, 1.0, 64), (256, 0.01, 128), (1024, 1.0, 128),
                                       (640, 0.5, 256)])
@pytest.mark.parametrize("int8", [True, False])
def test_sla2_infer_edge_shapes(L, topk, bq, int8):
    """One ragged block (L = 40), T = 1, every key block routed (an empty
    complement: the linear branch is 0 / eps), three batch rows."""
    from imfvideo_amd import ops
    say("sla2_infer edge L", L, "topk", topk, "bq", bq, "int8", int8)
    H = 2
    q, k, v = _inputs(140 + L, 3, H, L, torch.bfloat16)
    mq = -(-L // bq)
    lut, T = O.route_1d(q.float(), k.float(), topk, bq)
    g = torch.Generator().manual_seed(8)
    alpha = 0.1 + 0.8 * torch.rand(H, mq, generator=g)
    o = ops.sla2_infer(cuda(q), cuda(k), cuda(v), cuda(alpha), cuda(torch.as_tensor(lut)), bq,
                       use_int8=int8)
    torch.cuda.synchronize()
    ref = O.infer_1d(q.float(), k.float(), v.float(), alpha, lut, bq, int8=int8,
                     t16=torch.bfloat16)
    got = o.cpu().float()
    print(f"  T {T} o max {max_abs(got, ref['o']):.2e} rel {rel_l2(got, ref['o']):.2e}",
          flush=True)
    assert torch.isfinite(got).all()
    assert max_abs(got, ref["o"]) < TOL_MAX and rel_l2(got, ref["o"]) < TOL_REL
