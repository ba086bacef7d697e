"""Pins the CPU oracle against what the mathematics fixes (CPU only).

The reference ships no golden vectors for this path, so every oracle function
is checked here against an independent formulation: exact rationals, exact
small-integer sums, brute-force ordering, fp64 dense attention and
torch.func.jvp autodiff, finite differences and special cases.
"""
import math
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import sla2_oracle as O
from tests.helpers import from_bits16, make_inputs, max_abs, rel_l2

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- quantisation
def _round_half_away_exact(fr):
    a = abs(fr)
    f = math.floor(a)
    r = f + (1 if a - f >= Fraction(1, 2) else 0)
    return -r if fr < 0 else r


def test_quantize_known_answers():
    # amax = 127 -> s = fl32(127/127) + 1e-12 = 1.0 exactly, so x / s = x.
    x = np.zeros((1, 64, 64), np.float32)
    vals = [127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5, 0.49999997, 3.25, -0.0]
    x[0, 0, :len(vals)] = vals
    q, s = O.quantize_blocks(x)
    assert s.dtype == np.float32 and s[0, 0] == np.float32(1.0)
    expect = [127, 1, -1, 2, -2, 3, -3, 127, -127, 0, 3, 0]  # ties away from zero
    assert q[0, 0, :len(vals)].tolist() == expect


def test_quantize_zero_tile_and_ragged():
    x = np.zeros((2, 100, 64), np.float32)
    x[1, 70, 3] = -2.0  # second block of row 1 is ragged (36 rows)
    q, s = O.quantize_blocks(x)
    assert q.shape == (2, 100, 64) and s.shape == (2, 2)
    assert s[0, 0] == np.float32(1e-12) and not q[0].any()
    assert q[1, 70, 3] == -127 and s[1, 1] == np.float32(2.0) / np.float32(127) + np.float32(1e-12)


def test_quantize_matches_exact_rationals():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(3, 128, 64, generator=g) * 3).to(torch.bfloat16).float().numpy()
    q, s = O.quantize_blocks(x)
    for b in range(3):
        for blk in range(2):
            tile = x[b, blk * 64:(blk + 1) * 64]
            amax = Fraction(float(np.abs(tile).max()))
            sd = np.float32(float(np.abs(tile).max())) / np.float32(127)
            # fl32(amax / 127) is the correctly rounded quotient
            ulp = Fraction(float(np.spacing(sd)))
            assert abs(Fraction(float(sd)) - amax / 127) <= ulp / 2
            assert s[b, blk] == sd + np.float32(1e-12)
            sf = Fraction(float(s[b, blk]))
            qt = q[b, blk * 64:(blk + 1) * 64]
            flat_x, flat_q = tile.reshape(-1), qt.reshape(-1)
            for i in range(0, flat_x.size, 37):
                y32 = np.float32(flat_x[i]) / np.float32(s[b, blk])
                assert flat_q[i] == _round_half_away_exact(Fraction(float(y32)))
                assert abs(Fraction(float(flat_x[i])) - flat_q[i] * sf) <= sf / 2 * (1 + Fraction(1, 10**5))
            assert np.abs(qt).max() == 127


# --------------------------------------------------------------------- pooling
def test_pool_exact_small_integers():
    g = np.random.default_rng(0)
    x = (g.integers(-64, 64, size=(2, 3, 200, 64)) / 8.0).astype(np.float32)  # exact sums
    p = O.pool_tiles(x, 4, 200)
    for b in range(4):
        rows = x[..., b * 64:min(200, (b + 1) * 64), :].astype(np.float64)
        np.testing.assert_array_equal(p[..., b, :], rows.mean(-2).astype(np.float32))


def test_pool_and_projection_error_bound():
    g = np.random.default_rng(1)
    x = g.standard_normal((2, 256, 64)).astype(np.float32)
    proj = (np.eye(64) + 0.05 * g.standard_normal((64, 64))).astype(np.float32)
    p = O.pool_tiles(x, 4, 256)
    ref = x.astype(np.float64).reshape(2, 4, 64, 64).mean(2)
    bound = 64 * np.finfo(np.float32).eps * np.abs(x).reshape(2, 4, 64, 64).mean(2)
    assert (np.abs(p - ref) <= bound).all()
    pp = O.project_pool(p, proj)
    ref_pp = p.astype(np.float64) @ proj.astype(np.float64).T
    bound2 = 64 * np.finfo(np.float32).eps * (np.abs(p) @ np.abs(proj).T)
    assert (np.abs(pp - ref_pp) <= bound2).all()


# ------------------------------------------------------------------------ top-k
def _brute_topk(row, T):
    def key(i):
        v = float(row[i])
        return (0, 0.0, i) if math.isnan(v) else (1, -v, i)
    return sorted(range(len(row)), key=key)[:T]


def test_topk_brute_force_ties_nan_signed_zero():
    g = np.random.default_rng(2)
    for trial in range(40):
        n = int(g.integers(2, 60))
        row = g.integers(-4, 5, size=n).astype(np.float32) / 2  # many ties
        if trial % 5 == 0:
            row[g.integers(0, n)] = np.nan
        if trial % 7 == 0:
            row[row == 0] = -0.0
        T = int(g.integers(1, n + 1))
        got = O.topk_rows(row[None], T)[0].tolist()
        assert got == _brute_topk(row, T), (row, T)


def test_topk_matches_torch_values_without_ties():
    g = torch.Generator().manual_seed(3)
    pc = torch.randn(4, 6, 468, generator=g)
    got = O.topk_rows(pc.numpy(), 46)
    ref = torch.topk(pc, 46, dim=-1).indices.numpy()
    assert np.array_equal(np.sort(got, -1), np.sort(ref, -1))
    assert np.array_equal(got, ref)  # descending order, as torch's sorted topk


def test_route_matches_fp64_where_gap_allows():
    B, H, Np, P = 1, 3, 20, 0
    q, k, _ = make_inputs(4, B, H, Np * 64, tangent=False)
    lut, T, qp, kp = O.route(q.float(), k.float(), 0.25, Np, P)
    qd = q.double().reshape(B, H, Np, 64, 64).mean(3)
    kd = k.double().reshape(B, H, Np, 64, 64).mean(3)
    pc = (qd @ kd.transpose(-1, -2)).numpy() / 8.0
    checked = 0
    for idx in np.ndindex(B, H, Np):
        srt = np.sort(pc[idx])[::-1]
        if srt[T - 1] - srt[T] > 1e-5:
            assert set(lut[idx].tolist()) == set(np.argsort(-pc[idx])[:T].tolist())
            checked += 1
    assert checked > Np


def test_tile_permutation_round_trip():
    from imfvideo_amd.mla_video_sparse_jvp import tile_permutation
    perm, inv, n = tile_permutation((4, 8, 8), (2, 4, 4), 18, torch.device("cpu"))
    x = torch.randn(274, 5)
    assert torch.equal(x[perm][inv], x) and n == 8
    p2, i2, n2 = O.tile_permutation((4, 8, 8), (2, 4, 4), 18)
    assert np.array_equal(perm.numpy(), p2) and np.array_equal(inv.numpy(), i2) and n2 == 8
    # first tile = the 2x4x4 cube at the grid origin, prefix tokens last
    assert perm[:4].tolist() == [18, 19, 20, 21] and perm[16].item() == 18 + 64
    assert perm[-18:].tolist() == list(range(18))


# -------------------------------------------------------------- attention + JVP
def _case(seed=0, B=2, H=2, Np=4, P=18, topk=0.5, tan=1.0):
    L = Np * 64 + P
    q, k, v, dq, dk, dv = (t.float() for t in make_inputs(seed, B, H, L, tan_scale=tan))
    g = torch.Generator().manual_seed(seed + 7)
    alpha = torch.rand(H, -(-L // 64), generator=g) * 0.8 + 0.1
    lut, T, _, _ = O.route(q, k, topk, Np, P)
    return q, k, v, dq, dk, dv, alpha, lut, Np, P


def test_blockwise_matches_dense_fp64_jvp():
    q, k, v, dq, dk, dv, alpha, lut, Np, P = _case()
    ro, rdo = O.dense_jvp(q, k, v, dq, dk, dv, alpha, lut, Np, P)
    o, do = O.cube_jvp(q, k, v, dq, dk, dv, alpha, lut, Np, P, t16=torch.float32)
    assert rel_l2(o, ro) < 1e-5 and rel_l2(do, rdo) < 1e-5
    o, do = O.cube_jvp(q, k, v, dq, dk, dv, alpha, lut, Np, P, t16=torch.bfloat16)
    assert rel_l2(o, ro) < 1e-2 and rel_l2(do, rdo) < 1e-2
    assert max_abs(o, ro) < 2e-2 and max_abs(do, rdo) < 2e-2


def test_dense_jvp_matches_finite_differences():
    q, k, v, dq, dk, dv, alpha, lut, Np, P = _case(seed=1, B=1, H=1, Np=2, P=5, topk=0.5)
    L, D = q.shape[-2:]
    q8, qs = O.quantize_blocks(q)
    k8, ks = O.quantize_blocks(k)
    deq = lambda x8, s: torch.as_tensor(x8).double() * torch.as_tensor(s).double().repeat_interleave(64, -1)[..., :L, None]
    S = deq(q8, qs) @ deq(k8, ks).transpose(-1, -2) * D ** -0.5
    dS = (dq.double() @ k.double().transpose(-1, -2) + q.double() @ dk.double().transpose(-1, -2)) * D ** -0.5
    m, comp = O.block_mask(lut, Np, L, P)
    f = lambda eps: O.dense_op(S + eps * dS, v.double() + eps * dv.double(), q.double() + eps * dq.double(),
                               k.double() + eps * dk.double(), alpha, m, comp, Np)
    h = 1e-5
    fd = (f(h) - f(-h)) / (2 * h)
    _, do = O.dense_jvp(q, k, v, dq, dk, dv, alpha, lut, Np, P)
    assert rel_l2(do, fd) < 1e-6


def test_alpha_one_is_sparse_only_and_alpha_zero_linear_only():
    q, k, v, dq, dk, dv, alpha, lut, Np, P = _case(seed=2)
    H, Mb = alpha.shape
    ones, zeros = torch.ones(H, Mb), torch.zeros(H, Mb)
    o1, do1 = O.cube_jvp(q, k, v, dq, dk, dv, ones, lut, Np, P, t16=torch.float32)
    os_, dos = O.cube_jvp(q, k, v, dq, dk, dv, ones, lut, Np, P, t16=torch.float32, sparse_only=True)
    assert torch.equal(o1, os_) and torch.equal(do1, dos)
    # alpha = 0: linear branch only, against the dense fp64 complement form
    o0, _ = O.cube_jvp(q, k, v, dq, dk, dv, zeros, lut, Np, P, t16=torch.float32)
    m, comp = O.block_mask(lut, Np, q.shape[2], P)
    w = (torch.softmax(q.double(), -1) @ torch.softmax(k.double(), -1).transpose(-1, -2)) * comp
    ref = (w @ v.double()) / (w.sum(-1, keepdim=True) + O.EPS_L)
    assert rel_l2(o0, ref) < 1e-5


def test_all_tiles_routed_is_full_softmax():
    q, k, v, dq, dk, dv, alpha, _, Np, P = _case(seed=3, Np=3, P=10)
    B, H, L, D = q.shape
    lut = np.broadcast_to(np.arange(Np, dtype=np.int32), (B, H, 4, Np)).copy()
    ones = torch.ones(H, 4)
    o, _ = O.cube_jvp(q, k, v, dq, dk, dv, ones, lut, Np, P, t16=torch.float32)
    q8, qs = O.quantize_blocks(q)
    k8, ks = O.quantize_blocks(k)
    deq = lambda x8, s: torch.as_tensor(x8).double() * torch.as_tensor(s).double().repeat_interleave(64, -1)[..., :L, None]
    S = deq(q8, qs) @ deq(k8, ks).transpose(-1, -2) * D ** -0.5
    ref = torch.softmax(S, -1) @ v.double()
    assert rel_l2(o, ref) < 1e-5
    # alpha < 1 with an empty complement stays finite (signed epsilon)
    o2, do2 = O.cube_jvp(q, k, v, dq, dk, dv, alpha[:, :4], lut, Np, P)
    assert torch.isfinite(o2).all() and torch.isfinite(do2).all()


def test_phi_states_sum_invariant():
    q, k, v, dq, dk, dv, *_ = _case(seed=4)
    st = O.phi_states(k, v, 4, dk, dv)
    assert torch.allclose(st["Hall"], st["Hb"].sum(2)) and torch.allclose(st["dzall"], st["dzb"].sum(2))
    # zb rows of phi sum to 64 per tile (softmax rows sum to one)
    assert torch.allclose(st["zb"].sum(-1), torch.full_like(st["zb"].sum(-1), 64.0), atol=1e-4)
    # dphi rows sum to zero
    assert st["dzb"].sum(-1).abs().max() < 1e-4


# ---------------------------------------------------------------- golden files
@pytest.mark.parametrize("name", ["ref_geom_bf16", "tiny_f16", "two_tails_bf16"])
def test_oracle_reproduces_golden(name):
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    dt = getattr(torch, str(z["dtype"]))
    ins = {n: from_bits16(z[n], dt).float() for n in ("q", "k", "v", "dq", "dk", "dv")}
    Np, P = int(z["Np"]), int(z["P"])
    pq = torch.from_numpy(z["proj_q"]) if "proj_q" in z else None
    pk = torch.from_numpy(z["proj_k"]) if "proj_k" in z else None
    lut, T, qp, kp = O.route(ins["q"], ins["k"], float(z["topk"]), Np, P, pq, pk)
    assert np.array_equal(lut, z["lut"]) and np.array_equal(qp, z["qpool"]) and np.array_equal(kp, z["kpool"])
    q8, qs = O.quantize_blocks(ins["q"])
    assert np.array_equal(q8, z["q8"]) and np.array_equal(qs, z["qs"])
    o, do = O.cube_jvp(*(ins[n] for n in ("q", "k", "v", "dq", "dk", "dv")),
                       torch.from_numpy(z["alpha"]), lut, Np, P, t16=dt)
    assert max_abs(o, torch.from_numpy(z["o"])) < 1e-5 and max_abs(do, torch.from_numpy(z["do"])) < 1e-4


# ------------------------------------------------ training forward, semantics (b)
@pytest.mark.parametrize("path", ["train_fwd", "infer_1d"])
def test_int8_p_law_recovered_through_identity_values(path):
    """P enters the INT8 P.V product as trunc(127 p + 0.5) (reference
    models/sla2_vendor/kernel_sparse_qat.py:103, the truncating cast of a
    non-negative value), p = exp2(s - m) against the running maximum.  With
    V = 127 I (its INT8 tile is 127 I and its scale exactly 1), o_s = P8 / l
    row by row, so round(o_s * l) recovers every P8 exactly (16-bit o_s:
    relative error <= 2^-9, 127 * 2^-9 < 0.5).  The expected P8 comes from
    fp64 scores of the INT8 operands (their quantisation is pinned above);
    entries within 1e-3 of a rounding boundary are left out.  floor(127 p),
    a plausible slip, differs on about half of the entries."""
    g = torch.Generator().manual_seed(11)
    L, D = 64, 64
    q = torch.randn(1, 1, L, D, generator=g).to(torch.bfloat16).float()
    k = torch.randn(1, 1, L, D, generator=g).to(torch.bfloat16).float()
    v = torch.zeros(1, 1, L, D)
    v[0, 0, torch.arange(D), torch.arange(D)] = 127.0
    lut = np.zeros((1, 1, 1, 1), dtype=np.int32)
    if path == "train_fwd":
        res = O.train_fwd(q, k, v, torch.ones(1, 1), lut, 1, 0)
    else:
        res = O.infer_1d(q, k, v, torch.ones(1, 1), lut, 64)
    q8, qs = O.quantize_blocks_trunc(q)
    k8, ks = O.quantize_blocks_trunc(k)
    _, vs = O.quantize_blocks_trunc(v)
    assert float(vs[0, 0, 0]) == 1.0
    si = q8[0, 0].astype(np.float64) @ k8[0, 0].astype(np.float64).T
    c2 = float(np.float32(np.float32(D ** -0.5) * O.LOG2E))
    qk = si * float(qs[0, 0, 0]) * float(ks[0, 0, 0]) * c2
    p = np.exp2(qk - qk.max(1, keepdims=True))
    l = p.sum(1, keepdims=True)
    got = np.rint(res["o_s"][0, 0].double().numpy() * l)
    x = 127.0 * p + 0.5
    want = np.floor(x)
    keep = np.abs(x - np.rint(x)) > 1e-3
    assert keep.mean() > 0.95
    assert np.array_equal(got[keep], want[keep])
    assert (np.floor(127.0 * p) != want)[keep].mean() > 0.4


def test_quantize_trunc_known_answers():
    # amax = 127 -> s = 1 exactly (1e-12 vanishes in fp32): q = trunc(fl(x + 0.5 sign x))
    x = np.zeros((64, 64), np.float32)
    x[0, 0] = 127.0
    x[0, 1] = np.float32(0.49999997)   # + 0.5 rounds (to even) to 1.0 in fp32 -> 1
    x[0, 2] = -np.float32(0.49999997)  # -> -1
    x[0, 3] = 2.5
    x[0, 4] = -2.5
    x[0, 5] = -0.0
    x[0, 6] = np.float32(2.4999998)    # + 0.5 = 2.9999998 exactly -> 2
    q, s = O.quantize_blocks_trunc(x)
    assert s[0] == np.float32(1.0)
    assert q[0, :7].tolist() == [127, 1, -1, 3, -3, 0, 2]
    # round-half-away (the JVP path's quantiser) differs exactly on the first pair
    qa, _ = O.quantize_blocks(x)
    assert qa[0, :7].tolist() == [127, 0, 0, 3, -3, 0, 2]


def _train_case(seed=5, B=1, H=2, Np=4, P=18, topk=0.5):
    L = Np * 64 + P
    q, k, v, *_ = (t.float() for t in make_inputs(seed, B, H, L))
    g = torch.Generator().manual_seed(seed + 7)
    alpha = torch.rand(H, -(-L // 64), generator=g) * 0.8 + 0.1
    lut, T, _, _ = O.route(q, k, topk, Np, P)
    return q, k, v, alpha, lut, Np, P


def _dense_quantized_scores(q, k):
    """log2-domain scores from the (b) INT8 integers, dense, fp64."""
    L, D = q.shape[-2:]
    q8, qs = O.quantize_blocks_trunc(q)
    k8, ks = O.quantize_blocks_trunc(k)
    rep = lambda s: torch.as_tensor(s).double().repeat_interleave(64, -1)[..., :L]
    si = torch.as_tensor(q8).double() @ torch.as_tensor(k8).double().transpose(-1, -2)
    c2 = float(np.float32(np.float32(D ** -0.5) * O.LOG2E))
    return si * rep(qs)[..., :, None] * rep(ks)[..., None, :] * c2


def test_train_fwd_lse_is_dense_log2sumexp2():
    q, k, v, alpha, lut, Np, P = _train_case()
    r = O.train_fwd(q, k, v, alpha, lut, Np, P, t16=torch.float32)
    S = _dense_quantized_scores(q, k)
    m, _ = O.block_mask(lut, Np, q.shape[2], P)
    S = S.masked_fill(m == 0, -math.inf)
    ref = torch.logsumexp(S * math.log(2.0), -1) / math.log(2.0)
    assert (r["lse"].double() - ref).abs().max() < 1e-4


def test_train_fwd_sparse_branch_within_int8_p_bound():
    q, k, v, alpha, lut, Np, P = _train_case(seed=6)
    L = q.shape[2]
    r = O.train_fwd(q, k, v, alpha, lut, Np, P, t16=torch.float32)
    S = _dense_quantized_scores(q, k)
    m, _ = O.block_mask(lut, Np, L, P)
    Pm = torch.softmax((S * math.log(2.0)).masked_fill(m == 0, -math.inf), -1)
    v8, vs = O.quantize_blocks_trunc(v)
    vdq = torch.as_tensor(v8).double() * torch.as_tensor(vs).double().repeat_interleave(64, -1)[..., :L, None]
    ref = Pm @ vdq
    # P enters as trunc(127 p + 0.5) / 127 against the running maximum: a few per cent
    assert rel_l2(r["o_s"], ref) < 3e-2
    # a wrong scale, rescale or V factor is an O(1) error
    assert rel_l2(r["o_s"] * 1.1, ref) > 5e-2


def test_train_fwd_linear_branch_and_mix_endpoints():
    q, k, v, alpha, lut, Np, P = _train_case(seed=7)
    H, Mb = alpha.shape
    r1 = O.train_fwd(q, k, v, torch.ones(H, Mb), lut, Np, P, t16=torch.float32)
    r0 = O.train_fwd(q, k, v, torch.zeros(H, Mb), lut, Np, P, t16=torch.float32)
    assert torch.equal(r1["o"], r1["o_s"]) and torch.equal(r0["o"], r0["o_l"])
    # the linear branch is the (a) path's (pinned by its dense complement form)
    ol_a, _ = O.cube_jvp(q, k, v, None, None, None, torch.zeros(H, Mb), lut, Np, P, t16=torch.float32)
    assert rel_l2(r0["o_l"], ol_a) < 1e-5
    # 16-bit rounding of phi, the states and the outputs stays at bf16 level
    rb = O.train_fwd(q, k, v, alpha, lut, Np, P, t16=torch.bfloat16)
    rf = O.train_fwd(q, k, v, alpha, lut, Np, P, t16=torch.float32)
    assert rel_l2(rb["o"], rf["o"]) < 1e-2


def test_train_fwd_score_form_is_the_state_form_up_to_rounding():
    """The two forms of the linear branch are one sum regrouped: without 16-bit
    rounding they agree to fp32 precision (and with the dense complement of the
    (a) path); the 16-bit rounding points differ, so with bf16 they differ at
    bf16 level only.  The form follows the reference's switch, an augmented LUT
    of at most 4 columns (here T = 2 plus one prefix tail)."""
    q, k, v, alpha, lut, Np, P = _train_case(seed=8)
    H, Mb = alpha.shape
    zero = torch.zeros(H, Mb)
    sf = O.train_fwd(q, k, v, zero, lut, Np, P, t16=torch.float32, score_form=True)
    tf = O.train_fwd(q, k, v, zero, lut, Np, P, t16=torch.float32, score_form=False)
    ol_a, _ = O.cube_jvp(q, k, v, None, None, None, zero, lut, Np, P, t16=torch.float32)
    assert rel_l2(sf["o_l"], tf["o_l"]) < 1e-5 and rel_l2(sf["o_l"], ol_a) < 1e-5
    assert (sf["den"] - tf["den"]).abs().max() < 1e-4 * tf["den"].abs().max()
    sb = O.train_fwd(q, k, v, alpha, lut, Np, P, t16=torch.bfloat16, score_form=True)
    tb = O.train_fwd(q, k, v, alpha, lut, Np, P, t16=torch.bfloat16, score_form=False)
    assert not torch.equal(sb["o_l"], tb["o_l"])
    assert rel_l2(sb["o_l"], tb["o_l"]) < 1e-2
    # a dropped score term (one selected tile not subtracted) is an O(1) error
    lut1 = torch.as_tensor(np.asarray(lut))[..., :1]
    s1 = O.train_fwd(q, k, v, zero, lut1, Np, P, t16=torch.float32, score_form=True)
    assert rel_l2(s1["o_l"], sf["o_l"]) > 1e-2
    # the default follows the width of the augmented LUT
    auto = O.train_fwd(q, k, v, alpha, lut, Np, P, t16=torch.bfloat16)
    assert lut.shape[-1] + 1 <= 4 and torch.equal(auto["o"], sb["o"])
    wide = O.route(q, k, 1.0, Np, P)[0]                       # T = 4, 5 columns with the tail
    auto_w = O.train_fwd(q, k, v, alpha, wide, Np, P, t16=torch.bfloat16)
    state_w = O.train_fwd(q, k, v, alpha, wide, Np, P, t16=torch.bfloat16, score_form=False)
    assert torch.equal(auto_w["o"], state_w["o"])


def _bwd_case(seed, B=1, H=2, Np=3, P=10, T=2, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    L = Np * 64 + P
    nb = -(-L // 64)
    q, k, v, do = (torch.randn(B, H, L, 64, generator=g, dtype=torch.float64) for _ in range(4))
    q, k = q * 1.5, k * 1.5
    logit = torch.randn(H, nb, generator=g, dtype=torch.float64)
    lut = torch.stack([torch.randperm(Np, generator=g)[:T] for _ in range(B * H * nb)])
    lut = lut.view(B, H, nb, T).int().numpy()
    return q, k, v, do, logit, lut, Np, P


def test_train_bwd_exact_mode_is_the_autograd_gradient():
    # exact mode of the STE backward, fed the exact forward quantities, must be
    # the float64 autograd gradient of the unquantised op: pins every sign,
    # index and transpose of the sparse, linear, mix and phi-chain terms
    for seed in (0, 1):
        q, k, v, do, logit, lut, Np, P = _bwd_case(seed)
        xs = [t.clone().requires_grad_() for t in (q, k, v, logit)]
        o, fwd = O.train_dense_f64(*xs[:3], xs[3], lut, Np, P)
        want = torch.autograd.grad((o * do).sum(), xs)
        got = O.train_bwd(q, k, v, torch.sigmoid(logit), lut, Np, P, fwd, do, t16=None)
        for name, w in zip(("dq", "dk", "dv", "d_alpha"), want):
            err = ((got[name] - w).norm() / w.norm()).item()
            assert err < 1e-10, (seed, name, err)


def test_train_bwd_exact_mode_detects_a_planted_error():
    q, k, v, do, logit, lut, Np, P = _bwd_case(2)
    xs = [t.clone().requires_grad_() for t in (q, k, v, logit)]
    o, fwd = O.train_dense_f64(*xs[:3], xs[3], lut, Np, P)
    want = torch.autograd.grad((o * do).sum(), xs)
    bad = dict(fwd, ztot=fwd["ztot"] * 1.001)   # a perturbed linear-branch global
    got = O.train_bwd(q, k, v, torch.sigmoid(logit), lut, Np, P, bad, do, t16=None)
    err = ((got["dq"] - want[0]).norm() / want[0].norm()).item()
    assert err > 1e-6


def test_train_bwd_rounded_mode_near_exact_gradient():
    # 16-bit inputs, INT8 forward, 16-bit roundings and the STE: close to the
    # exact gradient of the unquantised op, at the INT8 level
    q, k, v, do, logit, lut, Np, P = _bwd_case(3)
    q16, k16, v16 = (t.to(torch.bfloat16).double() for t in (q, k, v))
    do16 = (do * 0.1).to(torch.bfloat16).double()
    xs = [t.clone().requires_grad_() for t in (q16, k16, v16, logit)]
    o, _ = O.train_dense_f64(*xs[:3], xs[3], lut, Np, P)
    want = torch.autograd.grad((o * do16).sum(), xs)
    a = torch.sigmoid(logit).float()
    f = [t.float() for t in (q16, k16, v16)]
    fwd = O.train_fwd(*f, a, lut, Np, P)
    got = O.train_bwd(*f, a, lut, Np, P, fwd, do16.float(), t16=torch.bfloat16)
    for name, w in zip(("dq", "dk", "dv", "d_alpha"), want):
        err = ((got[name].double() - w).norm() / w.norm()).item()
        assert err < 5e-2, (name, err)


def _case_1d(seed, L, B=1, H=2, bq=128, frac=0.3):
    g = torch.Generator().manual_seed(seed)
    x = [torch.randn(B, H, L, 64, generator=g, dtype=torch.float64) for _ in range(3)]
    d = [torch.randn(B, H, L, 64, generator=g, dtype=torch.float64) * 0.1 for _ in range(3)]
    lut, T = O.route_1d(x[0].float(), x[1].float(), frac, bq)
    mq = -(-L // bq)
    alpha = torch.rand(H, mq, generator=g, dtype=torch.float64) * 0.8 + 0.1
    return x, d, lut, alpha


def test_jvp_1d_exact_mode_matches_dense_jvp():
    # the reference's own dense oracle (sla2_dense_ref) and torch.func.jvp of it
    for L, bq in ((512, 128), (583, 128), (640, 64)):
        x, d, lut, alpha = _case_1d(L, L, bq=bq)
        f = lambda q_, k_, v_: O.dense_1d_f64(q_, k_, v_, lut, alpha, bq)
        eo, edo = torch.func.jvp(f, tuple(x), tuple(d))
        o, do = O.jvp_1d(*x, *d, alpha, lut, bq, t16=None)
        assert ((o.double() - eo).norm() / eo.norm()).item() < 1e-6, L
        assert ((do.double() - edo).norm() / edo.norm()).item() < 1e-6, L


def test_jvp_1d_rounded_within_reference_fp16_tolerance():
    # tests/test_sla2_jvp.py:41-42 bounds for fp16 operands: o 2e-2, do 5e-2
    x, d, lut, alpha = _case_1d(3, 583)
    x16 = [t.half().double() for t in x]
    d16 = [t.half().double() for t in d]
    f = lambda q_, k_, v_: O.dense_1d_f64(q_, k_, v_, lut, alpha, 128)
    eo, edo = torch.func.jvp(f, tuple(x16), tuple(d16))
    o, do = O.jvp_1d(*[t.float() for t in x16], *[t.float() for t in d16], alpha.float(), lut, 128)
    ro = ((o.double() - eo).norm() / eo.norm()).item()
    rdo = ((do.double() - edo).norm() / edo.norm()).item()
    assert ro < 2e-2 and rdo < 5e-2, (ro, rdo)
    assert ro > 1e-6  # the 16-bit roundings are in effect


def test_route_1d_matches_brute_force_block_scores():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, 2, 583, 64, generator=g).half().float()
    k = torch.randn(1, 2, 583, 64, generator=g).half().float()
    lut, T = O.route_1d(q, k, 0.3, 128)
    assert lut.shape == (1, 2, 5, 3) and T == 3
    # fp64 block means and scores: the selection agrees wherever the gap is clear
    qb = torch.stack([q[:, :, i:i + 128].double().mean(2) for i in range(0, 583, 128)], 2)
    kb = torch.stack([k[:, :, i:i + 64].double().mean(2) for i in range(0, 583, 64)], 2)
    kb = kb - kb.mean(2, keepdim=True)   # smooth-k: a per-row constant shift of the scores
    pc = (qb @ kb.transpose(-1, -2)) * 0.125
    want = torch.topk(pc, T, -1).indices.sort(-1).values
    got = torch.from_numpy(lut).long().sort(-1).values
    srt = pc.sort(-1, descending=True).values
    clear = (srt[..., T - 1] - srt[..., T]) > 1e-5
    assert clear.any() and torch.equal(got[clear], want[clear])


def test_train_bwd_1d_exact_mode_is_the_autograd_gradient():
    # 128-row query blocks, every 64-row key block routable, ragged L
    g = torch.Generator().manual_seed(11)
    B, H, L, bq = 1, 2, 583, 128
    nb, mq = -(-L // 64), -(-L // bq)
    q, k, v, do = (torch.randn(B, H, L, 64, generator=g, dtype=torch.float64) for _ in range(4))
    logit = torch.randn(H, mq, generator=g, dtype=torch.float64)
    lut, T = O.route_1d(q.float(), k.float(), 0.3, bq)
    xs = [t.clone().requires_grad_() for t in (q, k, v, logit)]
    o, fwd = O.train_dense_f64(*xs[:3], xs[3], lut, nb, 0, bq=bq)
    want = torch.autograd.grad((o * do).sum(), xs)
    for variant in ("cube", "1d"):
        got = O.train_bwd(q, k, v, torch.sigmoid(logit), lut, nb, 0, fwd, do, t16=None, bq=bq,
                          variant=variant)
        for name, w in zip(("dq", "dk", "dv", "d_alpha"), want):
            err = ((got[name] - w).norm() / w.norm()).item()
            assert err < 1e-10, (variant, name, err)


def test_train_fwd_1d_sixteen_bit_matches_dense():
    # 16-bit scores and P: the sparse branch within fp16 rounding of the dense form
    g = torch.Generator().manual_seed(12)
    B, H, L, bq = 1, 2, 583, 128
    nb, mq = -(-L // 64), -(-L // bq)
    q, k, v = (torch.randn(B, H, L, 64, generator=g).half().float() for _ in range(3))
    lut, T = O.route_1d(q, k, 0.3, bq)
    ones = torch.ones(H, mq)
    got = O.train_fwd(q, k, v, ones, lut, nb, 0, t16=torch.float16, int8=False, bq=bq)
    o, fwd = O.train_dense_f64(q.double(), k.double(), v.double(), torch.full((H, mq), 30.0,
                               dtype=torch.float64), lut, nb, 0, bq=bq)
    r = ((got["o_s"].double() - fwd["o_s"]).norm() / fwd["o_s"].norm()).item()
    assert r < 3e-3, r
    assert (got["lse"].double() - fwd["lse"]).abs().max().item() < 1e-3


def _mla_params(seed, D=128, H=2, dq=64, dc=32, F_=96, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, dtype=dtype)
    lin = lambda o, i: rn(o, i) * 0.5 / math.sqrt(i)
    p = {"H": H, "dq": dq, "dc": dc, "dn": 32, "dr": 32, "dv": 64,
         "w_norm1": 1 + 0.1 * rn(D), "w_qa": lin(dq, D), "w_kva": lin(dc + 32, D),
         "w_qa_ln": 1 + 0.1 * rn(dq), "w_kva_ln": 1 + 0.1 * rn(dc), "w_qb": lin(H * 64, dq),
         "w_kvb": lin(H * 96, dc), "w_qnorm": 1 + 0.1 * rn(32), "w_knorm": 1 + 0.1 * rn(32),
         "w_out": lin(D, H * 64), "g_attn": 0.1 + 0.01 * rn(D), "w_og": lin(H * 64, D),
         "w_norm2": 1 + 0.1 * rn(D), "w_gate": lin(F_, D), "w_up": lin(F_, D),
         "w_down": lin(D, F_), "g_mlp": 0.1 + 0.01 * rn(D), "situ_beta": 4.0}
    return p, g


def test_mla_sublayer_jvp_exact_mode_is_torch_func_jvp():
    import math as _m  # noqa: F401
    p, g = _mla_params(1)
    B, S, D = 1, 100, 128
    h = torch.randn(B, S, D, generator=g, dtype=torch.float64)
    dh = torch.randn(B, S, D, generator=g, dtype=torch.float64)
    cos, sin = (t.double() for t in O_rope(S))
    f = lambda x: O.mla_attn_eager(x, p, cos, sin, 1e-6, O.dense_attn_f64)
    want, dwant = torch.func.jvp(f, (h,), (dh,))
    attn_jvp = lambda q, k, v, dq, dk, dv: torch.func.jvp(O.dense_attn_f64, (q, k, v), (dq, dk, dv))
    a, da = O.mla_attn_jvp(h, dh, p, cos, sin, 1e-6, attn_jvp, t16=None)
    assert ((a - want).norm() / want.norm()).item() < 1e-10
    assert ((da - dwant).norm() / dwant.norm()).item() < 1e-10
    fm = lambda x: O.mlp_eager(x, p, 1e-6)
    want, dwant = torch.func.jvp(fm, (h,), (dh,))
    m, dm = O.mlp_jvp(h, dh, p, 1e-6, t16=None)
    assert ((m - want).norm() / want.norm()).item() < 1e-10
    assert ((dm - dwant).norm() / dwant.norm()).item() < 1e-10
    # without the output gate
    p["w_og"] = None
    want, dwant = torch.func.jvp(f, (h,), (dh,))
    a, da = O.mla_attn_jvp(h, dh, p, cos, sin, 1e-6, attn_jvp, t16=None)
    assert ((da - dwant).norm() / dwant.norm()).item() < 1e-10


def test_mla_eager_matches_package_module():
    # the oracle's eager restatement is the package's MLAAttention / SwiGLU forward
    from imfvideo_amd.imf_dit_video import TransformerBlock
    torch.manual_seed(0)
    blk = TransformerBlock(128, 2, 64, 32, 32, 32, 64, mlp_ratio=0.75, situ_linear_beta=None)
    with torch.no_grad():
        for prm in blk.parameters():
            prm.add_(0.05 * torch.randn_like(prm))
    from imfvideo_amd.mla_jvp_fast import mla_params_from_block
    p = {k: (v.double() if torch.is_tensor(v) else v) for k, v in mla_params_from_block(blk).items()}
    blk = blk.double()
    g = torch.Generator().manual_seed(2)
    x = torch.randn(1, 100, 128, generator=g, dtype=torch.float64)
    cos, sin = (t.double() for t in O_rope(100))
    blk.attn.attn_impl = lambda q, k, v: O.dense_attn_f64(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)).transpose(1, 2)
    got = blk(x, cos, sin)   # RMSNorm and RoPE compute in fp32, as the reference's modules
    h1 = x + O.mla_attn_eager(x, p, cos, sin, 1e-6, O.dense_attn_f64)
    want = h1 + O.mlp_eager(h1, p, 1e-6)
    assert ((got - want).norm() / want.norm()).item() < 1e-6


def O_rope(S):
    from imfvideo_amd.imf_dit_video import precompute_axial_rope_3d
    return precompute_axial_rope_3d(32, (1, 10, 10), S - 100, axis_dims=(8, 12, 12))


# ---------------------------------------------------------------------------
# Inference forward of the 1-D SLA2 (infer_1d)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("block", [32, 128, 256])
def test_quantize_blocks_other_block_sizes_brute_force(block):
    g = torch.Generator().manual_seed(40 + block)
    x = (torch.randn(1, 2, 300, 64, generator=g) * 3).half().float()
    q, s = O.quantize_blocks(x, block)
    xn = x.numpy().astype(np.float64)
    for b in range(-(-300 // block)):
        rows = slice(b * block, min(300, (b + 1) * block))
        for h in range(2):
            am = np.float32(np.abs(x.numpy()[0, h, rows]).max())
            sb = np.float32(np.float32(am / np.float32(127.0)) + np.float32(1e-12))
            assert s[0, h, b] == sb
            for val, qv in zip(xn[0, h, rows].ravel()[::97], q[0, h, rows].ravel()[::97]):
                y = Fraction(float(np.float32(np.float32(val) / sb)))
                assert qv == _round_half_away_exact(y)


def _infer_case(seed, L, bq, dt=torch.float16):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, 2, L, 64, generator=g).to(dt).float() for _ in range(3))
    mq = -(-L // bq)
    lut, _ = O.route_1d(q, k, 0.3, bq)
    alpha = 0.1 + 0.8 * torch.rand(2, mq, generator=g)
    return q, k, v, lut, alpha


def test_infer_1d_sixteen_bit_matches_dense():
    q, k, v, lut, alpha = _infer_case(50, 583, 128)
    got = O.infer_1d(q, k, v, alpha, lut, 128, int8=False)
    want = O.dense_1d_f64(q.double(), k.double(), v.double(), lut, alpha.double(), 128)
    assert rel_l2(got["o"], want) < 1e-3
    assert max_abs(got["o"], want) < 2e-3


@pytest.mark.parametrize("bq,qblock", [(128, None), (128, 64), (64, 32)])
def test_infer_1d_int8_matches_dense_of_the_dequantised_operands(bq, qblock):
    # sparse branch on the dequantised Q8, K8, V8 (P8 adds <= 1/254 per weight),
    # linear branch on the raw 16-bit values, alpha mix
    L = 583
    q, k, v, lut, alpha = _infer_case(51, L, bq)
    qb = bq if qblock is None else qblock
    got = O.infer_1d(q, k, v, alpha, lut, bq, int8=True, qblock=qblock)
    deq = lambda x, blk: (torch.as_tensor(O.quantize_blocks(x, blk)[0]).double()
                          * torch.as_tensor(O.quantize_blocks(x, blk)[1]).double()
                          .repeat_interleave(blk, -1)[..., :L, None])
    qd, kd, vd = deq(q, qb), deq(k, 64), deq(v, 64)
    o_s = O.dense_1d_f64(qd, kd, vd, lut, torch.ones_like(alpha).double(), bq)
    o_l = O.dense_1d_f64(q.double(), k.double(), v.double(), lut,
                         torch.zeros_like(alpha).double(), bq)
    a = alpha.double().repeat_interleave(bq, -1)[:, :L].view(1, 2, L, 1)
    want = a * o_s + (1 - a) * o_l
    assert rel_l2(got["o_s"], o_s) < 2e-2
    assert rel_l2(got["o"], want) < 2e-2
    assert max_abs(got["o"], want) < 5e-2
    # all key blocks routed: no complement, the output is the sparse branch
    nb = -(-L // 64)
    full = torch.arange(nb).view(1, 1, 1, nb).expand(1, 2, -(-L // bq), nb)
    got1 = O.infer_1d(q, k, v, torch.ones_like(alpha), full, bq, int8=True, qblock=qblock)
    assert torch.equal(got1["o"], got1["o_s"])


@pytest.mark.parametrize("int8", [False, True])
def test_infer_1d_fused_is_the_unfused_op_up_to_rounding(int8):
    """The fused Algorithm-2 arithmetic regroups the same sums (the complement as
    whole-sequence state minus the selected tiles' scores) and keeps o_s in
    fp32: without 16-bit rounding it equals the unfused inference path to fp32
    precision, with fp16 it differs at fp16 level, and it matches the dense
    fp64 form as well as the unfused path does."""
    L, bq = 583, 128
    q, k, v, lut, alpha = _infer_case(53, L, bq)
    kw = dict(int8=int8, qblock=64 if int8 else None)
    f32 = O.infer_1d(q, k, v, alpha, lut, bq, t16=torch.float32, fused=True, **kw)
    u32 = O.infer_1d(q, k, v, alpha, lut, bq, t16=torch.float32, **kw)
    assert rel_l2(f32["o"], u32["o"]) < 1e-5
    f16 = O.infer_1d(q, k, v, alpha, lut, bq, fused=True, **kw)
    u16 = O.infer_1d(q, k, v, alpha, lut, bq, **kw)
    assert not torch.equal(f16["o"], u16["o"])
    assert rel_l2(f16["o"], u16["o"]) < 5e-3
    # o_s enters the mix unrounded: with alpha = 1 the output is round16(o_s fp32)
    one = O.infer_1d(q, k, v, torch.ones_like(alpha), lut, bq, fused=True, **kw)
    assert torch.equal(one["o"], one["o_s"])
    if not int8:
        want = O.dense_1d_f64(q.double(), k.double(), v.double(), lut, alpha.double(), bq)
        assert rel_l2(f16["o"], want) < 1e-3 and max_abs(f16["o"], want) < 2e-3
    # a dropped correction (one selected tile left in the complement) is an O(1) error
    lut1 = torch.as_tensor(np.asarray(lut))[..., :1]
    zero = torch.zeros_like(alpha)
    d1 = O.infer_1d(q, k, v, zero, lut1, bq, t16=torch.float32, fused=True, **kw)
    u1 = O.infer_1d(q, k, v, zero, lut, bq, t16=torch.float32, fused=True, **kw)
    assert rel_l2(d1["o"], u1["o"]) > 1e-2


@pytest.mark.parametrize("bq", [128, 256])
def test_train_fwd_1d_int8_matches_dense_of_the_dequantised_operands(bq):
    # INT8 1-D training forward: sparse branch on the truncation-law Q8 (scales
    # per bq rows), K8, V8; the linear branch on the raw 16-bit values
    L, H = 583, 2
    q, k, v, lut, alpha = _infer_case(52, L, bq)
    nb = -(-L // 64)
    got = O.train_fwd(q, k, v, alpha, lut, nb, 0, t16=torch.float16, int8=True, bq=bq)

    def deq(x, blk):
        x8, xs = O.quantize_blocks_trunc(x, blk)
        return (torch.as_tensor(x8).double()
                * torch.as_tensor(xs).double().repeat_interleave(blk, -1)[..., :L, None])
    o_s = O.dense_1d_f64(deq(q, bq), deq(k, 64), deq(v, 64), lut,
                         torch.ones_like(alpha).double(), bq)
    assert rel_l2(got["o_s"], o_s) < 2e-2
    # the Q scale runs per bq rows: with per-64-row scales the integer scores differ
    q8, _ = O.quantize_blocks_trunc(q, bq)
    q8_64, _ = O.quantize_blocks_trunc(q, 64)
    assert not np.array_equal(q8, q8_64)
