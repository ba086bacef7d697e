"""Benchmark: SLA2 INT8 cube attention fwd+JVP at N=29,952 on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config 3|2|1] [--cpu-baseline 0|1]

A step is one call of the whole op on resident inputs -- INT8 quantisation
+ router pooling, top-k routing, linear-branch states, complement records and
the fused attention kernel -- for the BASELINE Config 3 workload (B=1, H=8,
N=29,952, D=64, top-k 10% -> T=46, bf16 Q/K/V and tangents; Config 2 is the
primal-only run).  Per-kernel durations come from HIP events recorded on the
launch stream between the stages inside the timed region.  Prints one JSON line.
"""

import argparse
import hashlib
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "ms per SLA2 INT8 attn fwd+JVP @N=29,952 on 1 MI355X; % of i8-MFMA/HBM roofline"
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_I8_TOPS = 5000.0         # MI355X dense int8 MFMA
PEAK_HBM_GBS = 8000.0
STAGES = ["quant_pool", "route_topk", "linear_states", "complement", "fwd_jvp"]


SETTLE_MS = 150.0


def settle(step, min_ms=SETTLE_MS, max_steps=2000):
    """Untimed full steps until the GPU has run the workload for min_ms of
    wall time, before the --warmup steps.  The MI355X's clocks ramp up under
    sustained load: the Config 3 op's per-step time falls by about 15 % over
    its first ~40 steps (35-40 ms) and is flat after that, also after an idle
    pause, so a handful of warm-up steps would time part of the ramp rather
    than the steady state a training or serving loop runs at.  The first
    step's own time (one-time set-up) is not counted toward min_ms.  Returns
    what was run (reported in the JSON line as "settle")."""
    step()  # a first call may include one-time set-up (library handles, kernel loads)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 1
    while n < max_steps:
        step()
        n += 1
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= min_ms:
            break
    return {"ms": round((time.perf_counter() - t0) * 1e3, 1), "steps": n,
            "note": "untimed full steps before the --warmup steps: the GPU clock ramp"}


def make_config(cfg):
    """Inputs on the CPU generator (seeded as in the parity tests), then to the GPU."""
    if cfg == 1:
        B, H, N, Np, seed, rms = 1, 4, 4096, 64, 1, False
    else:
        B, H, N, Np, seed, rms = 1, 8, 29952, 468, 2, True
    g = torch.Generator().manual_seed(seed)
    x = [torch.randn(B, H, N, 64, generator=g) for _ in range(3)]
    if rms:
        for i in (0, 1):
            x[i] = x[i] * torch.rsqrt(x[i].pow(2).mean(-1, keepdim=True) + 1e-6)
    qkv = [t.to(torch.bfloat16) for t in x]
    g2 = torch.Generator().manual_seed(3 if cfg != 1 else 101)
    tan = [(torch.randn(B, H, N, 64, generator=g2) * 0.1).to(torch.bfloat16) for _ in range(3)]
    alpha = torch.full((H, Np), 0.9)
    return dict(B=B, H=H, N=N, Np=Np, qkv=qkv, tan=tan, alpha=alpha, topk=0.1)


def measured_traffic(cfg, tangent):
    """HBM bytes per fwd_jvp launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (scaled by the same counters on a plain copy kernel),
    for the Config 3 tangent workload only; None otherwise, and None when the
    record was measured on another kernel instance or another version of the
    kernel source (its sha256 is stored with the figures)."""
    path = os.path.join(ROOT, "profiles", "fwd_jvp_config3_traffic.json")
    if cfg != 3 or not tangent or not os.path.exists(path):
        return None
    with open(path) as f:
        rec = json.load(f)
    # the instance this run launches (bf16, tangent, linear branch, power-of-two scale)
    if rec.get("kernel") != "void sla2h::fwd_jvp_kernel<sla2h::BF16, true, true, true, false>(sla2h::FwdArgs)":
        return None
    src = os.path.join(ROOT, rec.get("source", "imfvideo_amd/csrc/attn.hip"))
    with open(src, "rb") as f:
        if hashlib.sha256(f.read()).hexdigest() != rec.get("source_sha256"):
            return None
    return int(rec["bytes_per_launch"])


def roofline_work(B, H, Mb, T, n_tail, tangent):
    pairs = B * H * Mb * (T + n_tail)
    ops_i8 = pairs * 2 * 64 ** 3
    flops16 = pairs * 2 * 64 ** 3 * (5 if tangent else 1)
    return pairs, ops_i8, flops16


def hbm_bytes(B, H, N, Np, tangent):
    """Algorithmic HBM bytes of quant_pool and linear_states (each tensor read
    or written once), plus the operand-tile writes of linear_states (the
    fragment-ordered kt / vt tiles fwd_jvp streams, a layout choice of this
    build): (quant, states, states_layout_writes)."""
    t = B * H * N * 64
    nb = -(-N // 64)
    quant = 2 * t * 2 + 2 * t + 2 * B * H * nb * 4 + B * H * (nb + Np) * 64 * 4
    n_in = 4 if tangent else 2
    states = n_in * t * 2 + (2 if tangent else 1) * B * H * Np * (64 * 64 + 64) * 4
    tile = B * H * nb * 64 * 64 * 2  # one 16-bit (64, 64) operand tile per block
    layout = (4 if tangent else 1) * tile  # K|dK and V|dV tiles, or V only
    return quant, states, layout


def complement_work(B, H, Mb, Np, T, tangent):
    """Algorithmic work of the complement stage: (read bytes, written bytes,
    MFMA flops).  Reads the tile states (Hb, zb; with the tangent dHb, dzb) and
    the LUT, writes the per-query-block records (Hc, zc; dHc, dzc); the 0/1-mask
    GEMM runs on bf16 MFMA with the states split hi + lo (two products) over
    the padded extents (query blocks to 16, tiles to 32)."""
    parts = 2 if tangent else 1
    read = parts * B * H * Np * (64 * 64 + 64) * 4 + B * H * Mb * T * 4
    write = parts * B * H * Mb * (64 * 64 + 64) * 4
    mp, npad = -(-Mb // 16) * 16, -(-Np // 32) * 32
    flops = 2 * 2 * B * H * mp * npad * parts * (64 * 64 + 64)
    return read, write, flops


PROBE_SRC = os.path.join(ROOT, "bench_stream_probe.hip")
PROBE_LIB = os.path.join(ROOT, "bench_stream_probe.so")


def build_probe():
    """Compile the streaming-ceiling kernel (measurement only, not part of the
    product library) into bench_stream_probe.so for gfx950."""
    import subprocess
    from imfvideo_amd import build as _b
    tmp = PROBE_LIB + ".tmp"
    res = subprocess.run([_b.hipcc(), *_b.COMMON_FLAGS, "-shared", PROBE_SRC, "-o", tmp],
                         stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building {PROBE_SRC} failed:\n{res.stdout}")
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def stream_ceiling(read_bytes, write_bytes):
    """Fastest time for the same read / write byte counts with a plain
    streaming kernel (bench_stream_probe.so: 16 B per lane, nontemporal, grid-stride;
    best of two grids and five runs), after a 1 GiB write that flushes L2 and
    the 256 MB MALL ('flushed') and with the inputs just read ('resident')."""
    import ctypes
    if not os.path.exists(PROBE_LIB):
        build_probe()
    lib = ctypes.CDLL(PROBE_LIB)
    lib.sla2h_probe_stream.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] + [ctypes.c_int] * 3 + [ctypes.c_void_p]
    if write_bytes == 0:
        rd, wr = 1, 0
    else:
        ratio = read_bytes / write_bytes
        rd, wr = min(((2, 1), (1, 1), (1, 2)), key=lambda m: abs(m[0] / m[1] - ratio))
    n_grp = (read_bytes + write_bytes) // (16 * (rd + wr))
    dev = torch.device("cuda:0")
    src = torch.empty(rd * n_grp * 4, dtype=torch.int32, device=dev).fill_(1)
    dst = torch.empty(wr * n_grp * 4, dtype=torch.int32, device=dev)
    sink = torch.empty(8192 * 4, dtype=torch.int32, device=dev)
    junk = torch.empty(256 * 1024 * 1024, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = {"flushed": 1e9, "resident": 1e9}
    for grid in (1024, 4096):
        for rep in range(6):
            for mode in ("flushed", "resident"):
                if mode == "flushed":
                    junk.fill_(rep)
                e0.record()
                rc = lib.sla2h_probe_stream(src.data_ptr(), dst.data_ptr(), sink.data_ptr(), n_grp,
                                            rd, wr, grid, stream)
                e1.record()
                torch.cuda.synchronize()
                if rc != 0:
                    raise RuntimeError(f"sla2h_probe_stream failed ({rc})")
                if rep:
                    best[mode] = min(best[mode], e0.elapsed_time(e1) * 1e3)
    moved = 16 * (rd + wr) * n_grp
    del src, dst, sink, junk
    return {"mix": f"read:write {rd}:{wr}", "bytes": moved,
            "flushed_us": round(best["flushed"], 2), "resident_us": round(best["resident"], 2),
            "flushed_GB/s": round(moved / best["flushed"] / 1e3, 1),
            "resident_GB/s": round(moved / best["resident"] / 1e3, 1)}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(cfg_d, tangent):
    """The CPU oracle on the whole workload (all heads): routing, quantisation,
    states and the blockwise op, median of 3 calls after 1 warm-up."""
    from oracle import sla2_oracle as O
    torch.set_num_threads(os.cpu_count() or 1)
    f = lambda t: t.float()
    q, k, v = (f(t) for t in cfg_d["qkv"])
    dq, dk, dv = (f(t) for t in cfg_d["tan"]) if tangent else (None, None, None)
    Np = cfg_d["Np"]

    def once():
        lut, T, _, _ = O.route(q, k, cfg_d["topk"], Np, 0)
        O.cube_jvp(q, k, v, dq, dk, dv, cfg_d["alpha"], lut, Np, 0)

    once()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    return {"value": statistics.median(times) * 1e3, "unit": "ms", "cores": torch.get_num_threads(),
            "cpu_model": cpu_model(), "kind": "port",
            "sample": f"oracle (eager torch/numpy fp32, route + quant + states + blockwise op) on "
                      f"the whole workload ({cfg_d['B']} x {cfg_d['H']} heads), median of 3 calls "
                      f"after 1 warm-up"}


def timed_steps(step, steps, n_events, after=None):
    """The timed region: `steps` back-to-back calls of step(None) between two
    events, with synchronisation on both sides (the reported ms per step).
    Then, untimed, `steps` more calls of step(ev) that record the n_events
    events of ev inside the step for the stage breakdown: an event between two
    kernels costs a few microseconds and keeps them from overlapping, so it
    stays out of the reported figure.  after() runs after every step.
    Returns (ms per step, per-step event lists)."""
    ev_new = lambda: torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start, end = ev_new(), ev_new()
    start.record()
    for _ in range(steps):
        step(None)
        if after is not None:
            after()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    evs = [[ev_new() for _ in range(n_events)] for _ in range(steps)]
    for i in range(steps):
        step(evs[i])
        if after is not None:
            after()
    torch.cuda.synchronize()
    return ms, evs


TRAIN_STAGES = ["route", "quant_train", "sparse_fwd_qat", "linear_states_qat", "complement",
                "linear_mix_qat", "bwd_prep", "complement_bwd", "bwd_dq", "bwd_dkdv"]


def train_bench(args):
    """Config 5's attention op as one training step: routing, the training
    forward and the straight-through backward (B=2, H=8, N=29,952, fp16 as
    the reference module casts).  Not the headline metric: prints its own line."""
    from imfvideo_amd import ops

    B, H, N, Np, topk = 2, 8, 29952, 468, 0.1
    g = torch.Generator().manual_seed(5)
    x = [torch.randn(B, H, N, 64, generator=g) for _ in range(4)]
    for i in (0, 1):
        x[i] = x[i] * torch.rsqrt(x[i].pow(2).mean(-1, keepdim=True) + 1e-6)
    dev = torch.device("cuda:0")
    q, k, v, do = (t.to(torch.float16).to(dev) for t in x)
    alpha = torch.full((H, Np), 0.9, device=dev)
    T = ops.topk_count(topk, Np)
    nb = -(-N // 64)
    lib = ops._lib.load()

    def step(ev=None):
        rec = (lambda i: ev[i].record()) if ev is not None else (lambda i: None)
        rec(0)
        _, _, _, _, qpool, kpool_t = ops.quant_pool_qk(q, k, Np)
        lut = ops.route_topk(qpool, kpool_t, T, 0.125)
        rec(1)
        qz = ops.quant_train(q, k, v)
        rec(2)
        o_s, lse, qphi = ops.sparse_fwd_qat(q, qz, lut, Np)
        rec(3)
        st = ops.linear_states_qat(k, v)
        rec(4)
        lut_aug = ops.augment_lut(lut, Np, nb - Np)
        comp = ops.complement(st, lut_aug, nb, check_ids=False)  # LUT from route_topk
        rec(5)
        o, o_l, den = ops.linear_mix_qat(qphi, comp, st["Hall"], o_s, alpha)
        rec(6)
        fwd = dict(o_s=o_s, o_l=o_l, lse=lse, den=den, qphi=qphi, Hall=st["Hall"], comp=comp,
                   lut_aug=lut_aug)
        grads = ops.train_bwd(q, k, v, alpha, fwd, do, stage_events=(
            None if ev is None else ev[6:10]))
        rec(10)
        return o, grads

    settled = settle(step)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ms, evs = timed_steps(step, args.steps, 11)
    stage_us = {name: statistics.mean(e[si].elapsed_time(e[si + 1]) for e in evs) * 1e3
                for si, name in enumerate(TRAIN_STAGES)}
    pairs = B * H * nb * T  # n_tail = 0 at this shape
    gemm = 2 * 64 ** 3
    work = {"sparse_fwd_qat": ("int8", pairs * 2 * gemm), "bwd_dq": ("bf16", pairs * 3 * gemm),
            "bwd_dkdv": ("bf16", pairs * 4 * gemm)}
    roof = {}
    for kname, (kind, w) in work.items():
        peak = PEAK_I8_TOPS if kind == "int8" else PEAK_BF16_TFLOPS
        ach = w / (stage_us[kname] * 1e-6) / 1e12
        roof[kname] = {"bound": "mfma", "achieved": round(ach, 2), "peak": peak,
                       "unit": "TOP/s" if kind == "int8" else "TFLOP/s",
                       "frac": round(ach / peak, 4), "work": w}
    out = {
        "metric": "ms per SLA2 INT8 attn training step (fwd + straight-through bwd), "
                  "Config 5 attention shape, 1 MI355X",
        "value": round(ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle": settled, "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8+fp16",
        "data": "synthetic (CPU-seeded N(0,1); q,k per-token RMS-normalised; do N(0,1))",
        "config": {"workload": "SLA2 INT8 cube attention training step (BASELINE Config 5 "
                               "attention op)", "B": B, "H": H, "N": N, "D": 64, "E": 64,
                   "topk": topk, "T": T, "pairs": pairs},
        "roofline": roof,
        "kernels_us": {k_: round(v_, 2) for k_, v_ in stage_us.items()},
    }
    print(json.dumps(out), flush=True)


def block_step_bench(args):
    """Config 5: 8 stacked DiT blocks (RMSNorm -> MLA attention with the SLA2
    INT8 cube op -> SwiGLU MLP, ReZero scales 0.1), d=512, H=8, dq=256, dc=128,
    dn=dr=32, dv=64, MLP ratio 4, weights N(0, 0.5/sqrt(d_in)), B=2 x N=29,952
    tokens (12x48x52 grid kept tile-major, 4x4x4 tiles, top-k 10%).  One step:
    the forward with autograd (bf16 autocast), the fast forward + JVP pass
    (block_jvp from each block's pack_block snapshot, rebuilt every step as the
    weights change), and the backward of a loss that uses the JVP output only
    under stop-gradient (as iMF's does).  Prints its own line: ms per block."""
    from functools import partial
    from imfvideo_amd.imf_dit_video import TransformerBlock, precompute_axial_rope_3d
    from imfvideo_amd.mla_jvp_fast import block_jvp, pack_block
    from imfvideo_amd.mla_video_sparse_jvp import tile_permutation
    from imfvideo_amd.sla2_cube_qat import SLA2CubeQATAttentionImpl

    B, S, D, H, depth, grid = 2, 29952, 512, 8, 8, (12, 48, 52)
    dev = torch.device("cuda:0")
    torch.manual_seed(5)
    impl = partial(SLA2CubeQATAttentionImpl, seq_len=S, num_heads=H, grid=grid, tile=(4, 4, 4),
                   topk=0.1, pre_permuted=True)
    blocks = torch.nn.ModuleList(
        [TransformerBlock(D, H, 256, 128, 32, 32, 64, mlp_ratio=4, weight_init_constant=0.5,
                          attn_impl=impl) for _ in range(depth)]).to(dev)
    with torch.no_grad():
        for b in blocks:
            b.attn_scale.fill_(0.1)
            b.mlp_scale.fill_(0.1)
    perm, _, _ = tile_permutation(grid, (4, 4, 4), 0, torch.device("cpu"))
    cos, sin = (t[perm].to(dev) for t in precompute_axial_rope_3d(32, grid, 0,
                                                                  axis_dims=(8, 12, 12)))
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, S, D, generator=g).to(torch.bfloat16).float().to(dev)
    dx = (0.1 * torch.randn(B, S, D, generator=g)).to(dev)

    def step(ev=None):
        rec = (lambda i: ev[i].record()) if ev is not None else (lambda i: None)
        rec(0)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            h = x
            for b in blocks:
                h = b(h, cos, sin)
        rec(1)
        with torch.no_grad():
            hj, dhj = x, dx
            for b in blocks:
                pk, w16 = pack_block(b, tile_major=True)
                hj, dhj = block_jvp(hj, dhj, pk, w16, cos, sin, 1e-6)
        rec(2)
        loss = (h.float() - dhj).pow(2).mean()
        loss.backward()
        rec(3)
        return loss

    def step_zero():
        step()
        blocks.zero_grad(set_to_none=True)

    settled = settle(step_zero)
    for _ in range(args.warmup):
        step_zero()
    torch.cuda.synchronize()
    losses = []

    def step_keep(ev):
        losses.append(step(ev))

    ms, evs = timed_steps(step_keep, args.steps, 4, after=lambda: blocks.zero_grad(set_to_none=True))
    loss = losses[-1]
    st = {name: statistics.mean(e[k].elapsed_time(e[k + 1]) for e in evs) / depth
          for k, name in enumerate(["forward", "fast_jvp", "backward"])}
    print(json.dumps({
        "metric": "ms per DiT block (fwd + fast JVP + bwd) of an 8-block SLA2-INT8 stack, "
                  "BASELINE Config 5, 1 MI355X",
        "value": round(ms / depth, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle": settled, "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 autocast + int8/fp16 attention",
        "data": "synthetic (CPU-seeded x bf16 N(0,1), dx 0.1 N(0,1); weights N(0, 0.5/sqrt(d_in)))",
        "config": {"workload": "8 stacked DiT blocks, training step with the du/dt JVP "
                               "(BASELINE Config 5)", "B": B, "N": S, "d": D, "H": H,
                   "dq": 256, "dc": 128, "mlp_ratio": 4, "depth": depth, "topk": 0.1,
                   "tile_major": True},
        "loss": float(loss.item()),
        "per_block_ms": {k_: round(v_, 3) for k_, v_ in st.items()}}), flush=True)


def mla_bench(args):
    """Config 4: the MLA attention sublayer (sla2_mla_jvp variant) forward + JVP at
    N=29,952, d=512, H=8, dq=256, dc=128, dn=dr=32, dv=64, partial axial RoPE
    (8,12,12) over the 12x48x52 grid, weights N(0, 0.5/sqrt(d_in)), x ~ N(0,1)
    rounded to bf16, dx = 0.1 N(0,1), top-k 10% of 64-row key blocks with
    128-row query blocks.  Prints its own JSON line."""
    import math
    from imfvideo_amd.imf_dit_video import precompute_axial_rope_3d
    from imfvideo_amd.mla_jvp_fast import attn_sublayer_jvp, mla_fp16_cache

    B, S, D, H, dq, dc = 1, 29952, 512, 8, 256, 128
    g = torch.Generator().manual_seed(4)
    dev = torch.device("cuda:0")
    lin = lambda o, i: (torch.randn(o, i, generator=g) * 0.5 / math.sqrt(i)).to(dev)
    ones = lambda n: torch.ones(n, device=dev)
    p = {"H": H, "dq": dq, "dc": dc, "dn": 32, "dr": 32, "dv": 64, "w_norm1": ones(D),
         "w_qa": lin(dq, D), "w_kva": lin(dc + 32, D), "w_qa_ln": ones(dq), "w_kva_ln": ones(dc),
         "w_qb": lin(H * 64, dq), "w_kvb": lin(H * 96, dc), "w_qnorm": ones(32),
         "w_knorm": ones(32), "w_out": lin(D, H * 64), "g_attn": ones(D), "w_og": lin(H * 64, D),
         "w_norm2": ones(D), "w_gate": lin(8, D), "w_up": lin(8, D), "w_down": lin(D, 8),
         "g_mlp": ones(D)}
    mq = -(-S // 128)
    p["sla2"] = {"alpha": torch.full((H, mq), 0.9, device=dev), "proj_q": None, "proj_k": None,
                 "topk": 0.1, "bq": 128, "bk": 64}
    w16 = mla_fp16_cache(p)
    x = torch.randn(B, S, D, generator=g).to(torch.bfloat16).float().to(dev)
    dx = (0.1 * torch.randn(B, S, D, generator=g)).to(dev)
    cos, sin = (t.to(dev) for t in precompute_axial_rope_3d(32, (12, 48, 52), 0, axis_dims=(8, 12, 12)))
    settled = settle(lambda: attn_sublayer_jvp(x, dx, p, w16, cos, sin, 1e-6))
    for _ in range(args.warmup):
        attn_sublayer_jvp(x, dx, p, w16, cos, sin, 1e-6)
    torch.cuda.synchronize()
    def step(ev):
        if ev is None:
            return attn_sublayer_jvp(x, dx, p, w16, cos, sin, 1e-6)
        ev[0].record()
        return attn_sublayer_jvp(x, dx, p, w16, cos, sin, 1e-6, stage_events=ev[1:])

    ms, evs = timed_steps(step, args.steps, 4)
    st = {name: statistics.mean(e[k].elapsed_time(e[k + 1]) for e in evs) * 1e3
          for k, name in enumerate(["norm_gemms_head_prep", "sla2_mla_jvp", "gate_out_proj"])}
    print(json.dumps({
        "metric": "ms per MLA attention sublayer fwd+JVP (sla2_mla_jvp variant) @N=29,952, "
                  "1 MI355X", "value": round(ms, 4), "unit": "ms", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "settle": settled,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (CPU-seeded; weights N(0, 0.5/sqrt(d_in)); x bf16 N(0,1))",
        "config": {"workload": "MLA attention sublayer JVP (BASELINE Config 4)", "B": B, "N": S,
                   "d": D, "H": H, "dq": dq, "dc": dc, "bq": 128, "bk": 64, "topk": 0.1},
        "stages_us": {k_: round(v_, 2) for k_, v_ in st.items()}}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5],
                    help="4: the MLA sublayer JVP (own line); 5: the attention op's training "
                         "step at Config 5's shape (own line)")
    ap.add_argument("--cpu-baseline", type=int, default=1)
    ap.add_argument("--op-only", action="store_true",
                    help="Config 5: time the attention op's training step instead of the blocks")
    ap.add_argument("--hbm-ceiling", action="store_true",
                    help="print only the streaming ceilings (bench_stream_probe.so) for the read:write "
                         "mixes and byte counts of quant_pool and linear_states, one JSON line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 256 MiB fp32 copy kernel (torch.mul by 1) three times: "
                         "the reference reading for the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.copy_calibration:
        x = torch.randn(64 * 1024 * 1024, device="cuda")
        y = torch.empty_like(x)
        for _ in range(3):
            torch.mul(x, 1.0, out=y)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration": "256 MiB read + 256 MiB written per dispatch"}))
        return
    if args.hbm_ceiling:
        t_in = 8 * 29952 * 64 * 2  # one (1, 8, 29952, 64) 16-bit tensor
        cases = {"read only, 247 MB": (247283712, 0),
                 "read:write 1:1, 247 MB (linear_states, algorithmic)": (4 * t_in, 247283712 - 4 * t_in),
                 "read:write 2:1, 94 MB (quant_pool)": (2 * t_in, 93959424 - 2 * t_in),
                 "read:write 1:2, 370 MB (linear_states with operand tiles)": (4 * t_in, 369967104 - 4 * t_in),
                 "read:write 1:1, 1 GB": (500 << 20, 500 << 20)}
        print(json.dumps({name: stream_ceiling(r, w) for name, (r, w) in cases.items()}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the op shards by (batch, head) with no exchange between GPUs", file=sys.stderr)
        sys.exit(1)

    if args.config == 5:
        (train_bench if args.op_only else block_step_bench)(args)
        return
    if args.config == 4:
        mla_bench(args)
        return

    from imfvideo_amd import ops

    tangent = args.config in (1, 3)
    c = make_config(args.config)
    dev = torch.device("cuda:0")
    q, k, v = (t.to(dev) for t in c["qkv"])
    dq, dk, dv = (t.to(dev) for t in c["tan"]) if tangent else (None, None, None)
    alpha = c["alpha"].to(dev)
    Np, B, H, N = c["Np"], c["B"], c["H"], c["N"]
    T = ops.topk_count(c["topk"], Np)
    torch.cuda.synchronize()

    def step(ev=None):
        rec = (lambda i: ev[i].record()) if ev is not None else (lambda i: None)
        rec(0)
        q8, qs, k8, ks, qpool, kpool_t, kb = ops.quant_pool_qk(q, k, Np, with_kb=True)
        rec(1)
        lut = ops.route_topk(qpool, kpool_t, T, 0.125)
        rec(2)
        st = ops.linear_states(k, v, Np, dk, dv, with_sums=False)
        rec(3)
        comp = ops.complement(st, lut, Np, check_ids=False)
        rec(4)
        o, do = ops.fwd_jvp(q, q8, k8, qs, ks, st, comp, alpha, lut, Np, dq, kb=kb,
                            check_ids=False)
        rec(5)
        return o, do

    settled = settle(step)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ms, evs = timed_steps(step, args.steps, 6)
    stage_us = {}
    for si, name in enumerate(STAGES):
        stage_us[name] = statistics.mean(e[si].elapsed_time(e[si + 1]) for e in evs) * 1e3

    Mb = -(-N // 64)
    pairs, ops_i8, flops16 = roofline_work(B, H, Mb, T, Mb - Np, tangent)
    t_attn = stage_us["fwd_jvp"] * 1e-6
    achieved = (ops_i8 / 2 + flops16) / t_attn / 1e12
    qb, sb, sl = hbm_bytes(B, H, N, Np, tangent)
    # read / write split of each kernel's moved bytes for the matching ceiling
    t_in = B * H * N * 64 * 2
    q_read = 2 * t_in
    s_read = (4 if tangent else 2) * t_in
    ceil_q = stream_ceiling(q_read, qb - q_read)
    ceil_s = stream_ceiling(s_read, sb + sl - s_read)
    c_read, c_write, c_flops = complement_work(B, H, Mb, Np, T, tangent)
    ceil_c = stream_ceiling(c_read, c_write)

    def hbm_entry(name, alg, moved, ceil):
        us = stage_us[name]
        e = {"bytes": alg, "GB/s": round(alg / us / 1e3, 1),
             "frac": round(alg / us / 1e3 / PEAK_HBM_GBS, 4),
             "moved_bytes": moved, "moved_GB/s": round(moved / us / 1e3, 1),
             "ceiling": ceil, "frac_of_ceiling": round(ceil["flushed_us"] / us, 4)}
        if moved != alg:
            e["layout_write_bytes"] = moved - alg
        return e

    out = {
        "metric": METRIC,
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": settled,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8+bf16",
        "data": "synthetic (CPU-seeded N(0,1); q,k per-token RMS-normalised; tangents 0.1 N(0,1))",
        "config": {"workload": f"SLA2 INT8 cube attention {'fwd+JVP' if tangent else 'fwd'} "
                               f"(BASELINE Config {args.config})",
                   "B": B, "H": H, "N": N, "D": 64, "E": 64, "topk": c["topk"], "T": T,
                   "pairs": pairs},
        "roofline": {"bound": "mfma", "kernel": "fwd_jvp",
                     "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic(args.config, tangent),
                     "work": {"int8_ops": ops_i8, "bf16_flops": flops16,
                              "note": "achieved = (int8_ops/2 + bf16_flops) / t: int8 counted "
                                      "at its 2x peak, so frac = t_roofline / t"}},
        "kernels_us": {k_: round(v_, 2) for k_, v_ in stage_us.items()},
        "hbm_kernels": {
            "quant_pool": hbm_entry("quant_pool", qb, qb, ceil_q),
            "linear_states": hbm_entry("linear_states", sb, sb + sl, ceil_s),
            "complement": dict(hbm_entry("complement", c_read + c_write, c_read + c_write,
                                         ceil_c),
                               mfma={"bf16_flops": c_flops,
                                     "TFLOP/s": round(c_flops / stage_us["complement"] / 1e6, 2),
                                     "frac": round(c_flops / stage_us["complement"] / 1e6
                                                   / PEAK_BF16_TFLOPS, 4)}),
            "note": "bytes: algorithmic (each tensor once); frac: of 8 TB/s; ceiling: a "
                    "streaming kernel moving the same bytes at the same read:write mix; "
                    "frac_of_ceiling = flushed ceiling time / kernel time; complement: mask "
                    "and GEMM kernels together, mfma = the 0/1-mask GEMM's bf16 work (states "
                    "split hi + lo) against the dense bf16 peak",
        },
    }
    if args.cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(c, tangent)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
