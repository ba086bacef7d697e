"""The allocation-free complement entry point (sla2h_complement_noalloc, a
static per-GPU workspace instead of a caller-provided one) against
sla2h_complement, through the C ABI (marked gpu): records bit-identical on two
calls in a row, the second smaller (the static array keeps the first call's
masks, which the second must fully overwrite where it reads them), with and
without tangents; a workspace over the array's size is rejected."""
import pytest
import torch

from tests.helpers import make_inputs

pytestmark = pytest.mark.gpu


def _states(seed, B, H, Np, P, tangent):
    from imfvideo_amd import ops
    L = Np * 64 + P
    q, k, v, dq, dk, dv = (t.cuda() for t in make_inputs(seed, B, H, L))
    st = ops.linear_states(k, v, Np, dk if tangent else None, dv if tangent else None,
                           with_sums=False)
    Mb = -(-L // 64)
    T = max(1, Np // 7)
    g = torch.Generator().manual_seed(seed + 1)
    lut = torch.stack([torch.randperm(Np, generator=g)[:T] for _ in range(B * H * Mb)])
    return st, lut.view(B, H, Mb, T).to(torch.int32).cuda()


def _call(fn_name, st, lut, Np, ws=None):
    from imfvideo_amd import _lib, ops
    B, H, Mb, T = lut.shape
    lib = _lib.load()
    comp = torch.full((B, H, Mb, ops.REC_BYTES), 0xA5, device="cuda", dtype=torch.uint8)
    g = lambda n: ops._ptr(st.get(n))
    args = [g("Hb"), g("dHb"), g("zb"), g("dzb"), lut.data_ptr(), B, H, Mb, Np, 64, T]
    if ws is not None:
        args.append(ws.data_ptr())
    rc = getattr(lib, fn_name)(*args, comp.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0, (fn_name, rc)
    return comp


def test_noalloc_complement_matches_the_workspace_entry_point():
    from imfvideo_amd import _lib, ops
    lib = _lib.load()
    # the second call is smaller than the first: fewer heads, tiles and blocks
    for seed, B, H, Np, P, tan in ((3, 2, 8, 120, 40, True), (4, 1, 2, 13, 0, False),
                                   (5, 1, 3, 7, 100, True)):
        print(f"[case] noalloc complement B={B} H={H} Np={Np} P={P} tangent={tan}", flush=True)
        st, lut = _states(seed, B, H, Np, P, tan)
        Mb = lut.shape[2]
        ws = torch.empty(lib.sla2h_complement_workspace_bytes(B, H, Mb, Np), device="cuda",
                         dtype=torch.uint8)
        want = _call("sla2h_complement", st, lut, Np, ws)
        got = _call("sla2h_complement_noalloc", st, lut, Np)
        assert torch.equal(got, want)
        # through the Python wrapper (fresh torch.empty output: without tangents
        # only the Hc [0, 16384) and zc [32768, 33024) bytes of a record are written)
        via = ops.complement(st, lut, Np, noalloc=True)
        parts = [slice(0, ops.REC_BYTES)] if tan else [slice(0, 16384), slice(32768, 33024)]
        for sl in parts:
            assert torch.equal(via[..., sl], want[..., sl])
    # over the static array: rejected on the host, with real buffers large
    # enough for the claimed shape (B=1, H=3, Mb = Np = 4096 -> 6 MiB of masks)
    B, H, Np = 1, 3, 4096
    assert lib.sla2h_complement_workspace_bytes(B, H, Np, Np) > ops.COMPLEMENT_SCRATCH_BYTES
    Hb = torch.zeros(B, H, Np, 64, 64, device="cuda")
    zb = torch.zeros(B, H, Np, 64, device="cuda")
    lut = torch.zeros(B, H, Np, 1, device="cuda", dtype=torch.int32)
    comp = torch.empty(B, H, Np, ops.REC_BYTES, device="cuda", dtype=torch.uint8)
    rc = lib.sla2h_complement_noalloc(Hb.data_ptr(), None, zb.data_ptr(), None, lut.data_ptr(),
                                      B, H, Np, Np, 64, 1, comp.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == 1  # hipErrorInvalidValue
    with pytest.raises(ValueError, match="static"):
        ops.complement({"Hb": Hb, "zb": zb}, lut, Np, noalloc=True)
