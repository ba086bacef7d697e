"""CPU checks of the reference-facing Python API (no GPU): state-dict names and
shapes of the modules, the SoftTop-k router stage, and the torch-level helpers
of models/mla_video_sparse_jvp.py kept for the reference's tests
(_pool_tiles, _phi_jvp, _linear_jvp, mvs_dense_ref), each pinned by a closed
form or by the oracle's dense fp64 form."""
from functools import partial

import numpy as np
import pytest
import torch

from oracle import sla2_oracle as O
from tests.helpers import max_abs, rel_l2


# ---------------------------------------------------------------------------
# state dicts: the names and shapes checkpoints and the optimizer's parameter
# routing depend on (models/sla2_cube_qat.py:337-343, models/sla2_attention.py:
# 42-53, models/imf_dit_video.py:121-187, 377-421, 470-532, moonlight.py:506)
# ---------------------------------------------------------------------------
def test_cube_module_state_dict():
    from imfvideo_amd.sla2_cube_qat import SLA2CubeQATAttentionImpl
    mod = SLA2CubeQATAttentionImpl(head_dim=64, seq_len=274, num_heads=2, grid=(4, 8, 8),
                                   tile=(4, 4, 4), topk=0.5, alpha_init=0.9)
    sd = mod.state_dict()
    # perm / inv / a_index are non-persistent buffers: not in the checkpoint
    assert {k: tuple(v.shape) for k, v in sd.items()} == {
        "proj_q": (64, 64), "proj_k": (64, 64), "alpha_logit": (2, 5)}
    assert torch.equal(sd["proj_q"], torch.eye(64)) and torch.equal(sd["proj_k"], torch.eye(64))
    assert torch.allclose(torch.sigmoid(sd["alpha_logit"]), torch.full((2, 5), 0.9))
    assert (mod.Np, mod.E, mod.prefix_len, mod.n_tail, mod.Mb, mod.Nb) == (4, 64, 18, 1, 5, 5)
    assert mod.TILE_MAJOR is True and mod.use_int8 is True
    fresh = SLA2CubeQATAttentionImpl(head_dim=64, seq_len=274, num_heads=2, grid=(4, 8, 8))
    with torch.no_grad():
        mod.alpha_logit.add_(torch.randn(2, 5))
    fresh.load_state_dict(mod.state_dict(), strict=True)
    assert torch.equal(fresh.alpha_logit, mod.alpha_logit)
    assert [n for n, _ in mod.named_parameters()] == ["proj_q", "proj_k", "alpha_logit"]


def test_sla2_module_state_dict():
    from imfvideo_amd.sla2_attention import SLA2AttentionImpl
    mod = SLA2AttentionImpl(64, 583, 2, topk=0.3)
    assert {k: tuple(v.shape) for k, v in mod.state_dict().items()} == {
        "sla2.alpha_logit": (2, 5), "sla2.router.proj_q.weight": (64, 64),
        "sla2.router.proj_k.weight": (64, 64)}


def test_transformer_block_state_dict():
    from imfvideo_amd.imf_dit_video import TransformerBlock
    from imfvideo_amd.sla2_cube_qat import SLA2CubeQATAttentionImpl
    impl = partial(SLA2CubeQATAttentionImpl, seq_len=274, num_heads=2, grid=(4, 8, 8),
                   tile=(4, 4, 4), topk=0.5)
    blk = TransformerBlock(256, 2, 128, 64, 32, 32, 64, mlp_ratio=2, attn_impl=impl)
    want = {
        "norm1.weight": (256,), "norm2.weight": (256,), "attn_scale": (256,),
        "mlp_scale": (256,),
        "attn.q_a_proj.weight": (128, 256), "attn.q_b_proj.weight": (2 * 64, 128),
        "attn.kv_a_proj.weight": (64 + 32, 256), "attn.kv_b_proj.weight": (2 * (32 + 64), 64),
        "attn.out_proj.weight": (256, 2 * 64), "attn.g_proj.weight": (2 * 64, 256),
        "attn.q_a_layernorm.weight": (128,), "attn.kv_a_layernorm.weight": (64,),
        "attn.q_norm.weight": (32,), "attn.k_norm.weight": (32,),
        "attn.attn_impl.proj_q": (64, 64), "attn.attn_impl.proj_k": (64, 64),
        "attn.attn_impl.alpha_logit": (2, 5),
        "mlp.w1.weight": (512, 256), "mlp.w3.weight": (512, 256), "mlp.w2.weight": (256, 512),
    }
    assert {k: tuple(v.shape) for k, v in blk.state_dict().items()} == want
    # the optimizer routes alpha_logit by name (moonlight.py:506)
    assert any(n.endswith("alpha_logit") for n, _ in blk.named_parameters())


# ---------------------------------------------------------------------------
# SoftTop-k (models/sla2_vendor/router.py:23-45)
# ---------------------------------------------------------------------------
def test_soft_topk_row_sums_monotone_and_gradient():
    from imfvideo_amd.sla2_vendor.router import soft_topk
    g = torch.Generator().manual_seed(3)
    pc = torch.randn(2, 3, 7, 40, generator=g, dtype=torch.float64).float()
    for k_frac, tau in ((0.1, 0.1), (0.3, 0.5), (0.75, 0.05)):
        pcg = pc.clone().requires_grad_()
        s = soft_topk(pcg, k_frac, tau=tau)
        assert s.shape == pc.shape and (s >= 0).all() and (s <= 1).all()
        # each row sums to k_frac * Nb (bisection to 2e4 / 2^30 in lambda)
        assert torch.allclose(s.sum(-1), torch.full(s.shape[:-1], k_frac * 40), atol=2e-3)
        # monotone in the scores within a row
        order = pc.argsort(-1)
        ranked = torch.gather(s.detach(), -1, order)
        assert (ranked[..., 1:] >= ranked[..., :-1] - 1e-7).all()
        # lambda is detached: d(sum of row)/d(pc_ij) = sigmoid'(x_ij + lambda) / tau
        s.sum().backward()
        sd = s.detach().double()
        assert torch.allclose(pcg.grad.double(), sd * (1 - sd) / tau, rtol=1e-4, atol=1e-6)


# ---------------------------------------------------------------------------
# torch-level helpers of models/mla_video_sparse_jvp.py
# ---------------------------------------------------------------------------
def _cube_case(seed, B=2, H=2, Np=4, P=18, T=2, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    L = Np * 64 + P
    x = [torch.randn(B, H, L, 64, generator=g, dtype=torch.float64).to(dtype) for _ in range(6)]
    Mb = -(-L // 64)
    lut = torch.stack([torch.randperm(Np, generator=g)[:T] for _ in range(B * H * Mb)])
    lut = lut.view(B, H, Mb, T).to(torch.int32)
    alpha = (torch.rand(H, Mb, generator=g, dtype=torch.float64) * 0.8 + 0.1).to(dtype)
    return x, lut, alpha, Np, P


def test_pool_tiles_matches_the_oracle():
    from imfvideo_amd.mla_video_sparse_jvp import _pool_tiles
    g = torch.Generator().manual_seed(1)
    for Np, P in ((4, 18), (3, 64), (3, 130), (5, 0)):
        L = Np * 64 + P
        x = torch.randn(2, 2, L, 64, generator=g)
        got = _pool_tiles(x, Np, 64, P)
        nb = Np + -(-P // 64)
        assert got.shape == (2, 2, nb, 64)
        want = O.pool_tiles(x, nb, L)
        assert max_abs(got, torch.from_numpy(want)) < 1e-6


def test_phi_jvp_equals_torch_func_jvp_of_softmax():
    from imfvideo_amd.mla_video_sparse_jvp import _phi_jvp
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 3, 50, 64, generator=g, dtype=torch.float64)
    dx = torch.randn(2, 3, 50, 64, generator=g, dtype=torch.float64)
    phi, dphi = _phi_jvp(x, dx)
    p_ref, dp_ref = torch.func.jvp(lambda t: torch.softmax(t, -1), (x,), (dx,))
    assert max_abs(phi, p_ref) < 1e-6 and max_abs(dphi, dp_ref) < 1e-6


def test_linear_jvp_is_the_dense_form_at_alpha_zero():
    """alpha = 0 leaves only the linear branch, so mvs_dense_ref's tangent at
    alpha = 0 (torch.func.jvp, fp64) pins _linear_jvp's primal and tangent."""
    from imfvideo_amd.mla_video_sparse_jvp import _linear_jvp, _phi_jvp, mvs_dense_ref
    (q, k, v, dq, dk, dv), lut, alpha, Np, P = _cube_case(4)
    zero = torch.zeros_like(alpha)
    o_ref, do_ref = torch.func.jvp(lambda a, b, c: mvs_dense_ref(a, b, c, zero, lut, Np, 64, P),
                                   (q, k, v), (dq, dk, dv))
    qphi, dqphi = _phi_jvp(q, dq)
    kphi, dkphi = _phi_jvp(k, dk)
    o_l, do_l = _linear_jvp(qphi, dqphi, kphi, dkphi, v, dv, lut, Np, 64)
    assert rel_l2(o_l, o_ref) < 1e-6 and rel_l2(do_l, do_ref) < 1e-6
    o_p, none = _linear_jvp(qphi, dqphi, kphi, dkphi, v, dv, lut, Np, 64, primal_only=True)
    assert none is None and torch.equal(o_p, o_l)


def test_mvs_dense_ref_matches_the_oracle_dense_form():
    from imfvideo_amd.mla_video_sparse_jvp import mvs_dense_ref
    for P in (18, 0, 100):
        (q, k, v, _, _, _), lut, alpha, Np, _ = _cube_case(5 + P, P=P, Np=3)
        L = q.shape[2]
        got = mvs_dense_ref(q, k, v, alpha, lut, Np, 64, P)
        m, comp = O.block_mask(lut.numpy(), Np, L, P)
        S = (q @ k.transpose(-1, -2)) * 0.125
        want = O.dense_op(S, v, q, k, alpha, m, comp, Np)
        assert rel_l2(got, want) < 1e-12, P
    # alpha = 1 is the masked softmax; routing every tile makes it full attention
    (q, k, v, _, _, _), _, _, Np, P = _cube_case(9, T=4)
    L = q.shape[2]
    Mb = -(-L // 64)
    lut = torch.arange(Np, dtype=torch.int32).expand(2, 2, Mb, Np).contiguous()
    got = mvs_dense_ref(q, k, v, torch.ones(2, Mb, dtype=torch.float64), lut, Np, 64, P)
    full = torch.softmax((q @ k.transpose(-1, -2)) * 0.125, -1) @ v
    assert max_abs(got, full) < 1e-12


def test_mla_video_sparse_jvp_rejects_other_tile_lengths():
    import pytest
    from imfvideo_amd.mla_video_sparse_jvp import mla_video_sparse_jvp
    x = torch.zeros(1, 1, 8 * 32 + 18, 64)
    with pytest.raises(ValueError, match="tile length E must be 64"):
        mla_video_sparse_jvp(x, x, x, x, x, x, 0.5, 0.25, 8, 32, 18)


def test_fused_paths_fall_back_to_eager_for_unsupported_operands():
    """SituAndMul / the ReZero residual take the fused kernels only for GPU
    operands of the supported shapes and dtypes; here (CPU) they must equal the
    reference's eager expressions, including a broadcast scale and mixed dtypes."""
    from imfvideo_amd.imf_dit_video import SituAndMul, _residual
    g = torch.Generator().manual_seed(6)
    x = torch.randn(3, 5, 8, generator=g)
    a = torch.randn(3, 5, 8, generator=g)
    s1 = torch.randn(1, generator=g)
    assert torch.equal(_residual(x, a, s1), x + a * s1)
    gate = torch.randn(4, 16, generator=g, dtype=torch.float64)
    up = torch.randn(4, 16, generator=g).to(torch.bfloat16)
    act = SituAndMul(beta=4.0, linear_beta=25.0)
    gf, uf = gate.float(), up.float()
    want = (4.0 * torch.tanh(gf / 4.0) * torch.sigmoid(gf) * (25.0 * torch.tanh(uf / 25.0)))
    assert torch.equal(act(gate, up), want.to(torch.float64))
    np.testing.assert_array_equal(act(gate, up).numpy(), want.double().numpy())


def test_sla2_dense_ref_matches_the_oracle_dense_form():
    """models/sla2_mla_jvp.py:388-418's dense test utility against the oracle's
    fp64 restatement of the same form, ragged L and bq 64 / 128 / 256."""
    from imfvideo_amd.sla2_mla_jvp import sla2_dense_ref
    g = torch.Generator().manual_seed(8)
    for L, bq in ((583, 128), (512, 64), (640, 256)):
        q, k, v = (torch.randn(1, 2, L, 64, generator=g, dtype=torch.float64) for _ in range(3))
        mq, nb = -(-L // bq), -(-L // 64)
        T = max(1, nb // 3)
        lut = torch.stack([torch.randperm(nb, generator=g)[:T] for _ in range(2 * mq)])
        lut = lut.view(1, 2, mq, T).to(torch.int32)
        alpha = torch.rand(2, mq, generator=g, dtype=torch.float64) * 0.8 + 0.1
        got = sla2_dense_ref(q, k, v, lut, alpha, bq, 64)
        want = O.dense_1d_f64(q, k, v, lut.numpy(), alpha, bq)
        assert rel_l2(got, want) < 1e-12, (L, bq)


def test_alpha_reference_shape_with_a_long_prefix():
    """The reference's mix ratio alpha (H, Np + 1) has one column per video tile
    and one for the whole prefix, spread per token by repeat_interleave of
    [E] * Np + [P].  With a prefix of 150 tokens (three 64-row query blocks)
    alpha_blocks must give every prefix block that last column, and
    mvs_dense_ref must accept either form with the same result."""
    from imfvideo_amd.mla_video_sparse_jvp import alpha_blocks, mvs_dense_ref
    H, Np, P, E = 2, 3, 150, 64
    L = Np * E + P
    Mb = -(-L // E)
    g = torch.Generator().manual_seed(7)
    alpha_ref = torch.rand(H, Np + 1, generator=g)
    per_token = alpha_ref.repeat_interleave(torch.tensor([E] * Np + [P]), dim=1)  # (H, L)
    rows_of = torch.clamp(torch.arange(L) // E, max=Mb - 1)
    got = alpha_blocks(alpha_ref, H, Np, Mb, "cpu")
    assert got.shape == (H, Mb)
    assert torch.equal(got[:, rows_of], per_token)
    full = torch.rand(H, Mb, generator=g)
    assert torch.equal(alpha_blocks(full, H, Np, Mb, "cpu"), full)
    with pytest.raises(ValueError):
        alpha_blocks(torch.rand(H, Np), H, Np, Mb, "cpu")
    q, k, v = (torch.randn(1, H, L, 64, generator=g) for _ in range(3))
    lut = torch.stack([torch.randperm(Np, generator=g)[:2] for _ in range(H * Mb)]).view(1, H, Mb, 2)
    a = mvs_dense_ref(q, k, v, alpha_ref, lut, Np, E, P)
    b = mvs_dense_ref(q, k, v, got, lut, Np, E, P)
    assert torch.equal(a, b)


def test_caller_lut_ids_are_checked():
    """LUT ids outside [0, Np) (-1 padding, a prefix-tail id) are rejected before
    any kernel: the fused kernel would clamp them and the complement skip them."""
    from imfvideo_amd import ops
    lut = torch.tensor([[[[0, 3], [1, 2]]]], dtype=torch.int32)
    ops.check_lut_ids(lut, 4)
    for bad in (-1, 4):
        x = lut.clone()
        x[0, 0, 1, 0] = bad
        with pytest.raises(ValueError):
            ops.check_lut_ids(x, 4)
