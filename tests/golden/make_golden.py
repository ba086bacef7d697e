"""Write the small golden fixtures of this directory from the CPU oracle.

    python tests/golden/make_golden.py

Each case draws its inputs from a CPU torch.Generator, so the values are the
same on every host; the expected outputs come from oracle/sla2_oracle.py,
whose functions are pinned independently in tests/test_oracle.py.  The
reference ships no golden vectors for this path.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

from oracle import sla2_oracle as O  # noqa: E402
from helpers import bits16, make_inputs  # noqa: E402

CASES = {
    # the reference test geometry (tests/test_sla2_cube_qat.py:26-34), B=1, with
    # non-identity router projections as in tests/test_mla_video_sparse_jvp.py:43-44
    "ref_geom_bf16": dict(seed=10, B=1, H=2, Np=4, P=18, dtype=torch.bfloat16, topk=0.5,
                          proj=True),
    # fp16 storage, one routed tile, prefix of 40 tokens
    "tiny_f16": dict(seed=11, B=1, H=1, Np=3, P=40, dtype=torch.float16, topk=0.34, proj=False),
    # two prefix tail blocks, the last one ragged (6 rows)
    "two_tails_bf16": dict(seed=12, B=1, H=1, Np=2, P=70, dtype=torch.bfloat16, topk=0.5,
                           proj=False),
}


def build_case(seed, B, H, Np, P, dtype, topk, proj):
    L = Np * 64 + P
    q, k, v, dq, dk, dv = make_inputs(seed, B, H, L, dtype=dtype, tan_scale=1.0)
    g = torch.Generator().manual_seed(seed + 1000)
    Mb = -(-L // 64)
    alpha = torch.rand(H, Mb, generator=g) * 0.8 + 0.1
    pq = pk = None
    if proj:
        pq = torch.eye(64) + 0.05 * torch.randn(64, 64, generator=g)
        pk = torch.eye(64) + 0.05 * torch.randn(64, 64, generator=g)
    f = lambda t: t.float()
    lut, T, qp, kp = O.route(f(q), f(k), topk, Np, P, pq, pk)
    q8, qs = O.quantize_blocks(f(q))
    k8, ks = O.quantize_blocks(f(k))
    o, do = O.cube_jvp(f(q), f(k), f(v), f(dq), f(dk), f(dv), alpha, lut, Np, P,
                       quant=(q8, qs, k8, ks), t16=dtype)
    out = dict(dtype=np.array(str(dtype).split(".")[-1]), Np=np.array(Np), P=np.array(P),
               topk=np.array(topk), alpha=alpha.numpy(), lut=lut, q8=q8, qs=qs, k8=k8, ks=ks,
               qpool=qp, kpool=kp, o=o.numpy(), do=do.numpy())
    for name, t in zip(("q", "k", "v", "dq", "dk", "dv"), (q, k, v, dq, dk, dv)):
        out[name] = bits16(t)
    if proj:
        out["proj_q"] = pq.numpy()
        out["proj_k"] = pk.numpy()
    return out


def main():
    for name, cfg in CASES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **build_case(**cfg))
        print(path, os.path.getsize(path))


if __name__ == "__main__":
    main()
