"""GPU parity of the MLA attention-sublayer JVP, the MLP-sublayer JVP and the
block JVP (models/mla_jvp_fast.py:53-228) against the oracle's hand-propagated
restatement (O.mla_attn_jvp / O.mlp_jvp, pinned by torch.func.jvp of the eager
block).  Routing uses every key block (top-k fraction 1) so that 16-bit GEMM
rounding differences cannot change a LUT entry; the routed attention ops are
checked on their own elsewhere.  Tolerances: rel-L2 1e-2, max-abs 2e-2 of
max(1, max|ref|)."""
import math

import numpy as np
import pytest
import torch

from oracle import sla2_oracle as O
from tests.helpers import max_abs, rel_l2
from tests.test_gpu_parity import TOL_MAX, TOL_REL, cuda, say

pytestmark = pytest.mark.gpu


def params(seed, D=256, H=2, dq=128, dc=64, F_=512):
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g)
    lin = lambda o, i: rn(o, i) * 0.5 / math.sqrt(i)
    p = {"H": H, "dq": dq, "dc": dc, "dn": 32, "dr": 32, "dv": 64,
         "w_norm1": 1 + 0.1 * rn(D), "w_qa": lin(dq, D), "w_kva": lin(dc + 32, D),
         "w_qa_ln": 1 + 0.1 * rn(dq), "w_kva_ln": 1 + 0.1 * rn(dc), "w_qb": lin(H * 64, dq),
         "w_kvb": lin(H * 96, dc), "w_qnorm": 1 + 0.1 * rn(32), "w_knorm": 1 + 0.1 * rn(32),
         "w_out": lin(D, H * 64), "g_attn": 0.1 + 0.01 * rn(D), "w_og": lin(H * 64, D),
         "w_norm2": 1 + 0.1 * rn(D), "w_gate": lin(F_, D), "w_up": lin(F_, D),
         "w_down": lin(D, F_), "g_mlp": 0.1 + 0.01 * rn(D), "situ_beta": 4.0}
    return p, g


def gpu_params(p):
    return {k: (cuda(v) if torch.is_tensor(v) else v) for k, v in p.items()}


def rope(S, P):
    from imfvideo_amd.imf_dit_video import precompute_axial_rope_3d
    return precompute_axial_rope_3d(32, (4, 8, 8), P, axis_dims=(8, 12, 12))


def check(got, want, tag):
    for a, b, n in zip(got, want, ("out", "tangent")):
        a = a.cpu().double()
        b = b.double()
        bound = TOL_MAX * max(1.0, b.abs().max().item())
        print(f"  {tag} {n} max {max_abs(a, b):.2e} (bound {bound:.2e}) rel {rel_l2(a, b):.2e}",
              flush=True)
        assert max_abs(a, b) < bound and rel_l2(a, b) < TOL_REL


@pytest.mark.parametrize("path", ["dense", "sla2", "cube"])
def test_attn_sublayer_jvp(path):
    say("attn_sublayer_jvp", path)
    from imfvideo_amd.mla_jvp_fast import attn_sublayer_jvp, mla_fp16_cache
    from imfvideo_amd.mla_video_sparse_jvp import tile_permutation
    p, g = params(3)
    B, P = 2, 18
    S = 256 + P
    h = torch.randn(B, S, 256, generator=g)
    dh = 0.1 * torch.randn(B, S, 256, generator=g)
    cos, sin = rope(S, P)
    H = p["H"]
    nb = -(-S // 64)
    if path == "dense":
        lut = np.broadcast_to(np.arange(nb, dtype=np.int32), (B, H, nb, nb)).copy()
        ref_attn = lambda q, k, v, dq, dk, dv: O.jvp_1d(q, k, v, dq, dk, dv, torch.ones(H, nb),
                                                        lut, 64)
    elif path == "sla2":
        mq = -(-S // 128)
        alpha = torch.rand(H, mq, generator=g) * 0.8 + 0.1
        p["sla2"] = {"alpha": alpha, "proj_q": None, "proj_k": None, "topk": 1.0, "bq": 128,
                     "bk": 64}
        lut = np.broadcast_to(np.arange(nb, dtype=np.int32), (B, H, mq, nb)).copy()
        ref_attn = lambda q, k, v, dq, dk, dv: O.jvp_1d(q, k, v, dq, dk, dv, alpha, lut, 128)
    else:
        perm, inv, Np = tile_permutation((4, 8, 8), (4, 4, 4), P, torch.device("cpu"))
        alpha = torch.rand(H, nb, generator=g) * 0.8 + 0.1
        p["cube"] = {"alpha": alpha, "proj_q": None, "proj_k": None, "topk": 1.0, "Np": Np,
                     "E": 64, "P": P, "perm": perm, "inv": inv}
        lut = np.broadcast_to(np.arange(Np, dtype=np.int32), (B, H, nb, Np)).copy()

        def ref_attn(q, k, v, dq, dk, dv):
            t = lambda x: x[:, :, perm]
            o, do = O.cube_jvp(*(t(x) for x in (q, k, v, dq, dk, dv)), alpha, lut, Np, P,
                               t16=torch.float16)
            return o[:, :, inv], do[:, :, inv]
    pg = gpu_params(p)
    if "cube" in p:
        pg["cube"] = dict(p["cube"], alpha=cuda(alpha))
    if "sla2" in p:
        pg["sla2"] = dict(p["sla2"], alpha=cuda(alpha))
    a, da = attn_sublayer_jvp(cuda(h), cuda(dh), pg, mla_fp16_cache(pg), cuda(cos), cuda(sin), 1e-6)
    torch.cuda.synchronize()
    want = O.mla_attn_jvp(h, dh, p, cos, sin, 1e-6, ref_attn)
    check((a, da), want, path)


def test_mlp_and_block_jvp():
    say("mlp_sublayer_jvp, block_jvp (cube attention)")
    from imfvideo_amd.mla_jvp_fast import block_jvp, mla_fp16_cache, mlp_sublayer_jvp
    from imfvideo_amd.mla_video_sparse_jvp import tile_permutation
    p, g = params(4)
    B, P = 1, 18
    S = 256 + P
    h = torch.randn(B, S, 256, generator=g)
    dh = 0.1 * torch.randn(B, S, 256, generator=g)
    pg = gpu_params(p)
    w16 = mla_fp16_cache(pg)
    m, dm = mlp_sublayer_jvp(cuda(h), cuda(dh), pg, w16, 1e-6)
    check((m, dm), O.mlp_jvp(h, dh, p, 1e-6), "mlp")
    perm, inv, Np = tile_permutation((4, 8, 8), (4, 4, 4), P, torch.device("cpu"))
    nb = -(-S // 64)
    alpha = torch.full((p["H"], nb), 0.7)
    p["cube"] = {"alpha": alpha, "topk": 1.0, "Np": Np, "E": 64, "P": P, "perm": perm, "inv": inv}
    pg["cube"] = dict(p["cube"], alpha=cuda(alpha))
    cos, sin = rope(S, P)
    x, dx = block_jvp(cuda(h), cuda(dh), pg, w16, cuda(cos), cuda(sin), 1e-6)
    lut = np.broadcast_to(np.arange(Np, dtype=np.int32), (B, p["H"], nb, Np)).copy()

    def ref_attn(q, k, v, dq, dk, dv):
        t = lambda y: y[:, :, perm]
        o, do = O.cube_jvp(*(t(y) for y in (q, k, v, dq, dk, dv)), alpha, lut, Np, P,
                           t16=torch.float16)
        return o[:, :, inv], do[:, :, inv]
    a, da = O.mla_attn_jvp(h, dh, p, cos, sin, 1e-6, ref_attn)
    h1, dh1 = h + a, dh + da
    m, dm = O.mlp_jvp(h1, dh1, p, 1e-6)
    check((x, dx), (h1 + m, dh1 + dm), "block")


def _small_block(dev, attn_impl, seed=5):
    from imfvideo_amd.imf_dit_video import TransformerBlock
    torch.manual_seed(seed)
    blk = TransformerBlock(256, 2, 128, 64, 32, 32, 64, mlp_ratio=2, attn_impl=attn_impl)
    with torch.no_grad():
        blk.attn_scale.copy_(0.1 + 0.02 * torch.randn(256))
        blk.mlp_scale.copy_(0.1 + 0.02 * torch.randn(256))
        for n, prm in blk.named_parameters():
            if n.endswith("norm.weight") or n.endswith("layernorm.weight") or "norm1" in n \
                    or "norm2" in n:
                prm.add_(0.1 * torch.randn_like(prm))
    return blk.to(dev)


def _block_step(blk, x, w, cos, sin):
    xg = x.clone().requires_grad_()
    out = blk(xg, cos, sin)
    (out * w).sum().backward()
    return out.detach(), xg.grad


def _compare_blocks(gpu_blk, cpu_blk, got, want, rel, mx):
    from tests.block_ref import grad_report
    pairs = [("out", got[0], want[0]), ("x.grad", got[1], want[1])]
    pairs += [(f"grad {n}", a, b) for n, a, b in grad_report(gpu_blk, cpu_blk)]
    for tag, a, b in pairs:
        a, b = a.detach().cpu().double(), b.detach().cpu().double()
        bound = mx * max(1.0, b.abs().max().item())
        print(f"  {tag}: max {max_abs(a, b):.2e} (bound {bound:.2e}) rel {rel_l2(a, b):.2e}",
              flush=True)
        assert torch.isfinite(a).all() and max_abs(a, b) < bound and rel_l2(a, b) < rel, tag
    return len(pairs)


def test_transformer_block_training_step_dense_matches_eager():
    """The DiT block's training step with the fused GPU layers (RMSNorm,
    SituAndMul, RoPE on per-head and shared-key views, ReZero residuals)
    against the same block run eagerly on the CPU, dense attention, fp32:
    output, input gradient and every parameter gradient."""
    say("TransformerBlock (sdpa) fused GPU vs eager CPU: forward + backward")
    from imfvideo_amd.imf_dit_video import precompute_axial_rope_3d, sdpa_math_attention
    from tests.block_ref import copy_block_to_cpu
    S = 274
    blk = _small_block("cuda", sdpa_math_attention)
    ref = _small_block("cpu", sdpa_math_attention)
    copy_block_to_cpu(blk, ref)
    cos, sin = precompute_axial_rope_3d(32, (4, 8, 8), 18, axis_dims=(8, 12, 12))
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, S, 256, generator=g)
    w = torch.randn(2, S, 256, generator=g)
    got = _block_step(blk, cuda(x), cuda(w), cuda(cos), cuda(sin))
    want = _block_step(ref, x, w, cos, sin)
    n = _compare_blocks(blk, ref, got, want, rel=1e-4, mx=1e-4)
    assert n == 2 + 17  # every parameter of the block has a gradient


def test_transformer_block_training_step_cube_matches_oracle(monkeypatch):
    """The same block with SLA2CubeQATAttentionImpl (INT8 training forward,
    straight-through backward) against the eager CPU block whose attention is
    the oracle's training forward / backward (O.train_fwd / O.train_bwd) on
    the LUT the GPU block routed."""
    say("TransformerBlock (cube INT8) GPU vs eager CPU + oracle attention")
    from functools import partial
    import imfvideo_amd.sla2_cube_qat as cq
    from imfvideo_amd.imf_dit_video import precompute_axial_rope_3d
    from tests.block_ref import LutRecorder, OracleCubeAttention, copy_block_to_cpu
    S = 274
    kw = dict(seq_len=S, num_heads=2, grid=(4, 8, 8), tile=(4, 4, 4), topk=0.5)
    blk = _small_block("cuda", partial(cq.SLA2CubeQATAttentionImpl, **kw))
    with torch.no_grad():
        a = blk.attn.attn_impl.alpha_logit
        a.add_(torch.linspace(-1, 1, a.numel(), device="cuda").view_as(a))
    rec = LutRecorder(cq.route_tiles_fast)
    monkeypatch.setattr(cq, "route_tiles_fast", rec)
    ref = _small_block("cpu", partial(OracleCubeAttention, lut_source=lambda: rec.luts[-1], **kw))
    copy_block_to_cpu(blk, ref)
    cos, sin = precompute_axial_rope_3d(32, (4, 8, 8), 18, axis_dims=(8, 12, 12))
    g = torch.Generator().manual_seed(12)
    x = torch.randn(2, S, 256, generator=g)
    w = torch.randn(2, S, 256, generator=g)
    got = _block_step(blk, cuda(x), cuda(w), cuda(cos), cuda(sin))
    assert len(rec.luts) == 1
    want = _block_step(ref, x, w, cos, sin)
    _compare_blocks(blk, ref, got, want, rel=TOL_REL, mx=TOL_MAX)
    assert blk.attn.attn_impl.logit_max_log2.shape == (2,)


def test_pack_block_snapshot_drives_the_fast_jvp():
    """pack_block on a TransformerBlock with the cube attention: the snapshot
    (sigmoid(alpha_logit), projections, tiling) drives block_jvp, which then
    matches the oracle restatement fed the block's own weights."""
    say("pack_block (cube) -> block_jvp")
    from functools import partial
    from imfvideo_amd.imf_dit_video import TransformerBlock
    from imfvideo_amd.mla_jvp_fast import block_jvp, pack_block
    from imfvideo_amd.sla2_cube_qat import SLA2CubeQATAttentionImpl
    torch.manual_seed(6)
    S, P = 274, 18
    impl = partial(SLA2CubeQATAttentionImpl, seq_len=S, num_heads=2, grid=(4, 8, 8),
                   tile=(4, 4, 4), topk=1.0)
    blk = TransformerBlock(256, 2, 128, 64, 32, 32, 64, mlp_ratio=2, attn_impl=impl,
                           mla_use_output_gate=True).cuda()
    with torch.no_grad():
        blk.attn_scale.fill_(0.1)
        blk.mlp_scale.fill_(0.1)
        blk.attn.attn_impl.alpha_logit.copy_(torch.linspace(-1, 2, 2 * 5).view(2, 5))
    p, w16 = pack_block(blk)
    cube = p["cube"]
    assert torch.allclose(cube["alpha"], torch.sigmoid(blk.attn.attn_impl.alpha_logit.detach()))
    assert (cube["Np"], cube["E"], cube["P"], cube["topk"]) == (4, 64, P, 1.0)
    g = torch.Generator().manual_seed(8)
    h = torch.randn(1, S, 256, generator=g)
    dh = 0.1 * torch.randn(1, S, 256, generator=g)
    cos, sin = rope(S, P)
    x, dx = block_jvp(cuda(h), cuda(dh), p, w16, cuda(cos), cuda(sin), 1e-6)
    pc = {k: (v.detach().cpu().float() if torch.is_tensor(v) else v) for k, v in p.items()
          if k not in ("cube",)}
    perm, inv, Np = cube["perm"].cpu(), cube["inv"].cpu(), cube["Np"]
    alpha = cube["alpha"].cpu()
    nb = -(-S // 64)
    lut = np.broadcast_to(np.arange(Np, dtype=np.int32), (1, 2, nb, Np)).copy()

    def ref_attn(q, k, v, dq, dk, dv):
        t = lambda y: y[:, :, perm]
        o, do = O.cube_jvp(*(t(y) for y in (q, k, v, dq, dk, dv)), alpha, lut, Np, P,
                           t16=torch.float16)
        return o[:, :, inv], do[:, :, inv]
    a, da = O.mla_attn_jvp(h, dh, pc, cos, sin, 1e-6, ref_attn)
    h1, dh1 = h + a, dh + da
    m, dm = O.mlp_jvp(h1, dh1, pc, 1e-6)
    check((x, dx), (h1 + m, dh1 + dm), "packed block")


def test_build_fast_jvp_state_packs_every_block_of_a_net():
    """build_fast_jvp_state on a stand-in net with the reference model's
    attributes (two shared blocks, one u-head, the u-branch output layers,
    RoPE tables, eps, attention-residual block size, prefix tokens,
    tile_major): one pack_block per block in order, the u-branch tensors
    detached, the scalars passed through, and each packed block drives
    block_jvp to the same result as packing that block directly."""
    say("build_fast_jvp_state on a stand-in net")
    from functools import partial
    from types import SimpleNamespace
    from imfvideo_amd.imf_dit_video import TransformerBlock
    from imfvideo_amd.mla_jvp_fast import block_jvp, build_fast_jvp_state, pack_block
    from imfvideo_amd.sla2_cube_qat import SLA2CubeQATAttentionImpl
    torch.manual_seed(9)
    S, P, D = 274, 18, 256
    impl = partial(SLA2CubeQATAttentionImpl, seq_len=S, num_heads=2, grid=(4, 8, 8),
                   tile=(4, 4, 4), topk=0.5)
    mk = lambda: TransformerBlock(D, 2, 128, 64, 32, 32, 64, mlp_ratio=2, attn_impl=impl,
                                  mla_use_output_gate=True).cuda()
    blocks = [mk(), mk(), mk()]
    lin = torch.nn.Linear(D, 16).cuda()
    cos, sin = rope(S, P)
    net = SimpleNamespace(
        shared_blocks=blocks[:2], u_heads=blocks[2:], tile_major=False,
        u_out_res_norm=SimpleNamespace(weight=torch.nn.Parameter(torch.ones(D, device="cuda"))),
        u_out_res_proj=torch.nn.Linear(D, D, bias=False).cuda(),
        u_final_layer=SimpleNamespace(norm=SimpleNamespace(weight=torch.nn.Parameter(
            torch.ones(D, device="cuda"))), linear=lin),
        rope_cos=cuda(cos), rope_sin=cuda(sin), rmsnorm_eps=1e-6, attn_res_block_size=4,
        prefix_tokens=P)
    st = build_fast_jvp_state(net)
    assert len(st["shared"]) == 2 and len(st["u_heads"]) == 1
    assert st["eps"] == 1e-6 and st["bs"] == 4 and st["prefix_tokens"] == P
    assert st["rope"][0] is net.rope_cos and st["rope"][1] is net.rope_sin
    for t_ in (*st["u_out_res"], *st["u_final"]):
        assert not t_.requires_grad
    assert torch.equal(st["u_final"][1], lin.weight.detach())
    assert torch.equal(st["u_final"][2], lin.bias.detach())
    g = torch.Generator().manual_seed(10)
    h = cuda(torch.randn(1, S, D, generator=g))
    dh = cuda(0.1 * torch.randn(1, S, D, generator=g))
    for packed, blk in zip(st["shared"] + st["u_heads"], blocks):
        p1, w1 = packed
        p2, w2 = pack_block(blk, False)
        x1, dx1 = block_jvp(h, dh, p1, w1, cuda(cos), cuda(sin), 1e-6)
        x2, dx2 = block_jvp(h, dh, p2, w2, cuda(cos), cuda(sin), 1e-6)
        assert torch.equal(x1, x2) and torch.equal(dx1, dx2)
