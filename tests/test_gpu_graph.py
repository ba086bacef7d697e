"""The fused cube fwd+JVP op (quantisation, routing, states, complement,
attention) captured in one HIP graph: every replay, with eager calls of the op
and synchronisations between the replays, equals the eager result bit for bit
(the op records no memset and no host synchronisation, so a serving loop can
capture it).  Config 1's shape (B=1, H=4, N=4,096)."""
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_cube_jvp_graph_replays_match_eager():
    from imfvideo_amd import ops
    print("[case] graph capture of the fused op, Config 1 shape", flush=True)
    sys.stdout.flush()
    g = torch.Generator().manual_seed(11)
    B, H, N, Np = 1, 4, 4096, 64
    dev = torch.device("cuda:0")
    q, k, v = (torch.randn(B, H, N, 64, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    dq, dk, dv = ((0.1 * torch.randn(B, H, N, 64, generator=g)).to(torch.bfloat16).to(dev)
                  for _ in range(3))
    alpha = torch.full((H, Np), 0.9, device=dev)
    T = ops.topk_count(0.1, Np)

    def step():
        q8, qs, k8, ks, qpool, kpool_t, kb = ops.quant_pool_qk(q, k, Np, with_kb=True)
        lut = ops.route_topk(qpool, kpool_t, T, 0.125)
        st = ops.linear_states(k, v, Np, dk, dv, with_sums=False)
        comp = ops.complement(st, lut, Np, check_ids=False)
        return ops.fwd_jvp(q, q8, k8, qs, ks, st, comp, alpha, lut, Np, dq, kb=kb,
                           check_ids=False)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    torch.cuda.synchronize()
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        eo, edo = step()
        torch.cuda.synchronize()
        assert torch.equal(out[0], eo) and torch.equal(out[1], edo)
