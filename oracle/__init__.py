"""CPU oracle of the SLA2 INT8 cube-attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker or the reported CPU
baseline.  The product path (``imfvideo_amd``) never imports it and has no
CPU fallback.

Pinning status of each function (what checks it besides the GPU):
  quantize_blocks   closed form + exact-rational brute force (tests/test_oracle.py)
  pool_tiles        exact-sum cases + fp64 error bound
  project_pool      exact-sum cases + fp64 error bound
  route_scores      fp64 scores where the top-T gap exceeds rounding
  topk_rows         brute force over Python tuple sort; torch.topk value sets
  phi_states        dense einsum form + H_all = sum Hb invariant
  cube_jvp          dense fp64 masked-softmax form; torch.func.jvp of the dense
                    form (tangent); central finite differences; alpha = 0 / 1,
                    T = Np special cases
The reference ships no golden vectors for this path (all its tests draw
torch.randn on CUDA), so no reference-held fixture pins any function.
"""
