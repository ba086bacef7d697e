"""Tile geometry and the block router, with the reference's names and signatures.

Mirrors models/mla_video_sparse_jvp.py: ``tile_permutation`` (:61-91),
``route_tiles`` (:268-295), ``route_tiles_fast`` (:532-566) and
``_plenty_of_vram`` (:42-55).  Pooling, projections, scores and the top-k
run in the gfx950 kernels behind ``sla2h_quant_pool_qk`` and
``sla2h_route_topk`` with one pinned fp32 evaluation order, so the selected
tile sets are reproducible bit for bit.
"""

import torch

from . import ops

__all__ = ["tile_permutation", "route_tiles", "route_tiles_fast", "_plenty_of_vram"]


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

    q, k: (B, H, L, D) 16-bit tile-major.  Returns (lut (B,H,Mb,T) int32, T).
    Rows of the LUT are ordered by descending score (the reference returns
    them unordered, ``torch.topk(sorted=False)``).
    """
    B, H, L, D = q.shape
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
