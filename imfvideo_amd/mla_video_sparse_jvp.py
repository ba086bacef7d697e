"""Tile geometry, the block router and the non-QAT cube JVP, with the
reference's names and signatures (models/mla_video_sparse_jvp.py).

On the gfx950 kernels:
  ``route_tiles`` (:268-295) and ``route_tiles_fast`` (:532-566): pooling,
  projections, scores and the top-k behind ``sla2h_quant_pool_qk`` and
  ``sla2h_route_topk``, one pinned fp32 evaluation order, so the selected
  tile sets are reproducible bit for bit;
  ``mla_video_sparse_jvp`` (:403-454): the cube JVP with 16-bit primal
  scores (``ops.cube_jvp16``).
Host index math: ``tile_permutation`` (:61-91), ``_plenty_of_vram`` (:42-55).

The reference also exports four torch-level helpers that its tests import:
``_pool_tiles`` (:241-265), ``_phi_jvp`` (:301-308), ``_linear_jvp``
(:311-397) and the dense O(L^2) oracle ``mvs_dense_ref`` (:457-498).  They
are plain torch here as there, run on whatever device their inputs live on,
and no kernel path of this package calls them.
"""

import torch
import torch.nn.functional as F

from . import ops

__all__ = ["tile_permutation", "route_tiles", "route_tiles_fast", "_plenty_of_vram",
           "mla_video_sparse_jvp", "mvs_dense_ref", "_pool_tiles", "_phi_jvp", "_linear_jvp"]

_EPS_L = 1e-5


def _plenty_of_vram(device, need_gib=24.0):
    """True when `device` has more than `need_gib` GiB free (reference :42-55)."""
    try:
        free, _ = torch.cuda.mem_get_info(device)
        return free > need_gib * 2**30
    except Exception:  # noqa: BLE001 - CPU or query failure: be conservative
        return False


def tile_permutation(grid, tile, prefix_len, device):
    """Index maps between model order and tile-major order (reference :61-91).

    Model order: [prefix tokens (P)] + [patch tokens, t-major over grid].
    Tile order:  [patch tokens grouped by 3D tile] + [prefix tokens].

    Returns perm (L,) int64 with tile_tokens = model_tokens[perm],
    inv (L,) int64 with model_tokens = tile_tokens[inv], and Np.
    """
    T, Hh, Ww = grid
    tt, th, tw = tile
    assert T % tt == 0 and Hh % th == 0 and Ww % tw == 0, (grid, tile)
    idx = torch.arange(T * Hh * Ww, device=device).view(T // tt, tt, Hh // th, th, Ww // tw, tw)
    patch = idx.permute(0, 2, 4, 1, 3, 5).reshape(-1) + prefix_len
    perm = torch.cat([patch, torch.arange(prefix_len, device=device)])
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel(), device=device)
    return perm, inv, (T // tt) * (Hh // th) * (Ww // tw)


def _to16(x):
    return x if x.dtype in (torch.float16, torch.bfloat16) else x.to(torch.bfloat16)


def route_tiles_fast(q, k, topk_frac, Np, E, prefix_len, proj_q=None, proj_k=None):
    """Hard top-k router on pooled tiles (reference :532-566).

    q, k: (B, H, L, D) tile-major, 16-bit or fp32 (fp32 is pooled as given,
    unrounded).  Returns (lut (B,H,Mb,T) int32, T).  Rows of the LUT are
    ordered by descending score (the reference returns them unordered,
    ``torch.topk(sorted=False)``).
    """
    B, H, L, D = q.shape
    if q.dtype == torch.float32 and k.dtype == torch.float32:
        # the same pooling law (sequential fp32 row sums, / count, projection
        # as a sequential dot) on the unrounded inputs
        qpool = ops.pool_blocks(q, E, proj_q)
        kpool_t = ops.pool_blocks(k[:, :, :Np * E].contiguous(), E, proj_k, transposed=True)
    else:
        q, k = _to16(q), _to16(k)
        _, _, _, _, qpool, kpool_t = ops.quant_pool_qk(q, k.to(q.dtype), Np, E, proj_q, proj_k)
    T = ops.topk_count(topk_frac, Np)
    lut = ops.route_topk(qpool, kpool_t, T, D ** -0.5)
    return lut, T


def route_tiles(q, k, topk_frac, Np, E, prefix_len, proj_q=None, proj_k=None):
    """Router with smooth-k (reference :268-295).

    Subtracting the mean pooled key (before the optional projection) shifts
    every score row by a per-query constant, so the hard top-k selection is
    that of ``route_tiles_fast`` up to fp32 rounding; this build evaluates the
    shift-free form in the pinned order for both entry points.
    """
    return route_tiles_fast(q, k, topk_frac, Np, E, prefix_len, proj_q, proj_k)


# ---------------------------------------------------------------------------
# The non-QAT cube JVP (16-bit primal scores) on the gfx950 kernels.
# ---------------------------------------------------------------------------
def alpha_blocks(alpha, H, Np, Mb, device, dtype=torch.float32, detach=True):
    """Per-query-block mix ratios (H, Mb) fp32 from either form the callers use:
    (H, Mb) as given, or the reference's (H, Np + 1) -- one column per video
    tile and one shared by the whole prefix (its repeat_interleave of
    [E] * Np + [P], models/mla_video_sparse_jvp.py) -- whose last column covers
    every prefix block when the prefix spans more than one."""
    a = (alpha.detach() if detach else alpha).to(device, dtype)
    if a.dim() != 2 or a.shape[0] != H:
        raise ValueError(f"alpha: expected (H, Mb) or (H, Np + 1), got {tuple(a.shape)}")
    if a.shape[1] == Mb:
        return a
    if a.shape[1] == Np + 1 and Mb > Np:
        return torch.cat([a[:, :Np], a[:, Np:].expand(H, Mb - Np)], dim=1)
    raise ValueError(f"alpha: expected (H, {Mb}) or (H, {Np + 1}), got {tuple(a.shape)}")


def mla_video_sparse_jvp(q, k, v, dq, dk, dv, alpha, topk_frac, Np, E, prefix_len,
                         proj_q=None, proj_k=None, lut=None, T=None, block_m=64):
    """Cube-tile SLA2 attention and its forward-mode tangent, 16-bit scores.

    The exact branch attends, for every query block, the routed video tiles
    plus every prefix tail block; the linear branch takes the video tiles
    that were not routed (the prefix never enters it); the two are mixed by
    alpha per query block.  Inputs in tile order: Np tiles of E = 64 tokens
    and then the prefix_len conditioning tokens (L = Np * E + prefix_len).

    Args:
        q, k, v, dq, dk, dv: (B, H, L, 64) primal and tangent.  fp16 and bf16
            keep their type; fp32 inputs are routed as given but computed in
            fp16 (the reference's fp32 mode uses IEEE fp32 dots and meets
            o 2e-4 / do 2e-3 against the dense fp32 JVP; here fp32 inputs get
            the fp16 mode's precision, o ~1e-2).
        alpha: (H, Mb) mix after the sigmoid, or a scalar.
        topk_frac: routed fraction of the video tiles (unused with lut).
        Np, E, prefix_len: tiling geometry; E must be 64.
        proj_q, proj_k: optional (D, D) router projections.
        lut, T: precomputed routing (B, H, Mb, T), e.g. from a primal pass.
        block_m: accepted for the reference's signature (must divide E); the
            kernel's work unit is fixed.

    Returns:
        (o, do): (B, H, L, 64) fp32.
    """
    if E != ops.E_TILE:
        raise ValueError(f"mla_video_sparse_jvp: the tile length E must be {ops.E_TILE}, got {E}")
    if E % block_m:
        raise ValueError(f"block_m must divide E: {block_m}, {E}")
    B, H, L, D = q.shape
    if L != Np * E + prefix_len:
        raise ValueError(f"L={L} does not match Np={Np}, E={E}, prefix_len={prefix_len}")
    dt = q.dtype if q.dtype in (torch.float16, torch.bfloat16) else torch.float16
    qc, kc, vc, dqc, dkc, dvc = (t.to(dt).contiguous() for t in (q, k, v, dq, dk, dv))
    if lut is None:
        # routed on the inputs as given (fp32 unrounded), as the reference does
        lut, T = route_tiles(q.contiguous(), k.to(q.dtype).contiguous(), topk_frac, Np, E,
                             prefix_len, proj_q, proj_k)
    else:
        lut = lut.to(device=q.device, dtype=torch.int32).contiguous()
        ops.check_lut_ids(lut, Np)
    Mb = -(-L // E)
    if torch.is_tensor(alpha) and alpha.dim() == 2:
        a = alpha_blocks(alpha, H, Np, Mb, q.device)
    else:
        a = torch.full((H, Mb), float(alpha), device=q.device, dtype=torch.float32)
    return ops.cube_jvp16(qc, kc, vc, dqc, dkc, dvc, a, lut.to(q.device), Np)


# ---------------------------------------------------------------------------
# Torch-level helpers of the reference module (its tests import them).
# ---------------------------------------------------------------------------
def _pool_tiles(x, Np, E, prefix_cnt):
    """Tile means: (B, H, L, D) tile-major -> (B, H, Np + ceil(prefix_cnt / E), D)
    fp32; every video tile averages its E tokens, every prefix tail block the
    tokens it really holds (the last one may be short)."""
    B, H, L, D = x.shape
    xf = x.float()
    parts = [xf[:, :, :Np * E].reshape(B, H, Np, E, D).mean(dim=3)]
    start = Np * E
    while start < Np * E + prefix_cnt:
        parts.append(xf[:, :, start:min(start + E, L)].mean(dim=2, keepdim=True))
        start += E
    return torch.cat(parts, dim=2)


def _phi_jvp(x, dx):
    """phi(x) = softmax over the channel dim in fp32, and its tangent
    dphi = phi * (dx - <phi, dx>) -> (phi, dphi), both (B, H, L, D) fp32."""
    phi = torch.softmax(x.float(), dim=-1)
    dxf = dx.float()
    return phi, phi * (dxf - (phi * dxf).sum(dim=-1, keepdim=True))


def _linear_jvp(qphi, dqphi, kphi, dkphi, v, dv, lut, Np, E, primal_only=False):
    """Linear branch over the video tiles each query block did not route.

    For every query block m: H_c = sum over non-routed tiles n of
    phi(K_n)^T V_n and z_c = sum of phi(K_n) (prefix tokens excluded), then
    o_l = phi(q) H_c / (phi(q) . z_c + 1e-5), and its tangent by the product
    and quotient rules from the tangent states.  The routed part is summed
    one LUT column at a time and subtracted from the totals.

    Args:
        qphi, dqphi, kphi, dkphi, v, dv: (B, H, L, D) feature maps, values
            and their tangents (fp32 or 16-bit), tile-major.
        lut: (B, H, Mb, T) routed video-tile ids.
        Np, E: number of video tiles and tile length.
        primal_only: skip the tangent (returns None for it).

    Returns:
        (o_l, do_l): (B, H, L, D) fp32 (do_l None with primal_only).
    """
    B, H, L, D = qphi.shape
    Dv = v.shape[-1]
    Mb, T = lut.shape[2], lut.shape[3]
    tiles = lambda x, w: x.float()[:, :, :Np * E].reshape(B, H, Np, E, w)
    kt, vt = tiles(kphi, D), tiles(v, Dv)
    Hb = torch.einsum("bhntd,bhntv->bhndv", kt, vt)
    zb = kt.sum(dim=3)
    tan = not primal_only
    if tan:
        dkt, dvt = tiles(dkphi, D), tiles(dv, Dv)
        dHb = torch.einsum("bhntd,bhntv->bhndv", dkt, vt) + torch.einsum(
            "bhntd,bhntv->bhndv", kt, dvt)
        dzb = dkt.sum(dim=3)

    def complement(state):
        total = state.sum(dim=2, keepdim=True)
        routed = torch.zeros((B, H, Mb) + state.shape[3:], device=state.device,
                             dtype=state.dtype)
        idx = lut.long()
        for j in range(T):
            ix = idx[..., j].reshape(B, H, Mb, *([1] * (state.dim() - 3)))
            routed += torch.gather(state, 2, ix.expand((B, H, Mb) + state.shape[3:]))
        return total - routed

    Hc, zc = complement(Hb), complement(zb)
    pad = Mb * E - L
    qg = F.pad(qphi.float(), (0, 0, 0, pad)).reshape(B, H, Mb, E, D)
    num = torch.einsum("bhmtd,bhmdv->bhmtv", qg, Hc)
    den = torch.einsum("bhmtd,bhmd->bhmt", qg, zc) + _EPS_L
    o_l = num / den[..., None]
    flat = lambda x: x.reshape(B, H, Mb * E, x.shape[-1])[:, :, :L]
    if not tan:
        return flat(o_l), None
    dHc, dzc = complement(dHb), complement(dzb)
    dqg = F.pad(dqphi.float(), (0, 0, 0, pad)).reshape(B, H, Mb, E, D)
    dnum = (torch.einsum("bhmtd,bhmdv->bhmtv", dqg, Hc)
            + torch.einsum("bhmtd,bhmdv->bhmtv", qg, dHc))
    dden = (torch.einsum("bhmtd,bhmd->bhmt", dqg, zc)
            + torch.einsum("bhmtd,bhmd->bhmt", qg, dzc))
    do_l = (dnum - o_l * dden[..., None]) / den[..., None]
    return flat(o_l), flat(do_l)


def mvs_dense_ref(q, k, v, alpha, lut, Np, E, prefix_len):
    """Dense fp32 form of the cube op for tests (differentiable; O(L^2) memory).

    Token-level mask from the LUT (every routed video tile, plus the prefix
    columns for every query); exact branch = masked softmax attention with
    scale D^-1/2; linear branch = phi(q) phi(k)^T restricted to the video
    columns outside the mask, normalised by its row sum + 1e-5; mixed by
    alpha (H, Mb), one value per query block.

    Args: q, k, v (B, H, L, D) fp32 tile-major; alpha (H, Mb) or the
    reference's (H, Np + 1) (see alpha_blocks); lut
    (B, H, Mb, T); Np, E, prefix_len.  Returns o (B, H, L, D) fp32.
    """
    B, H, L, D = q.shape
    Mb = lut.shape[2]
    dev = q.device
    blocks = torch.zeros(B, H, Mb, Np, device=dev)
    blocks.scatter_(-1, lut.long(), 1.0)
    rows_of = torch.clamp(torch.arange(L, device=dev) // E, max=Mb - 1)
    cols_of = torch.clamp(torch.arange(Np * E, device=dev) // E, max=Np - 1)
    mask = blocks[:, :, rows_of][..., cols_of]                     # (B,H,L,Np*E)
    if L > Np * E:
        mask = torch.cat([mask, torch.ones(B, H, L, L - Np * E, device=dev)], dim=-1)
    scores = (q @ k.transpose(-1, -2)) * D ** -0.5
    o_s = torch.softmax(scores.masked_fill(mask <= 0, float("-inf")), dim=-1) @ v
    w = torch.softmax(q, dim=-1) @ torch.softmax(k, dim=-1).transpose(-1, -2)
    keep = 1.0 - mask
    keep[..., Np * E:] = 0.0
    w = w * keep
    o_l = (w @ v) / (w.sum(dim=-1, keepdim=True) + _EPS_L)
    a = alpha_blocks(alpha, H, Np, Mb, dev, dtype=q.dtype, detach=False)[:, rows_of].reshape(
        1, H, L, 1)
    return a * o_s + (1.0 - a) * o_l
