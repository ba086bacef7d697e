"""The C-ABI library: loads, exports every declared symbol, validates arguments (CPU)."""
import os
import re

import pytest
import torch

from imfvideo_amd import _lib, ops

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "sla2h.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sla2h_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    names = declared_symbols()
    assert len(names) >= 8
    assert names == sorted(_lib.SIGNATURES), "ctypes signatures must mirror include/sla2h.h"


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.sla2h_version() == 1
    assert lib.sla2h_complement_record_bytes(64) == ops.REC_BYTES
    assert lib.sla2h_complement_record_bytes(32) == 0


def test_invalid_arguments_are_rejected_before_any_launch():
    lib = _lib.load()
    bad = 1  # hipErrorInvalidValue
    assert lib.sla2h_quantize(None, 1, 1, 64, 64, 64, None, None, None) == bad
    assert lib.sla2h_quantize(1, 1, 1, 64, 32, 64, 1, 1, None) == bad       # D != 64
    assert lib.sla2h_quantize(1, 7, 1, 64, 64, 64, 1, 1, None) == bad       # dtype
    assert lib.sla2h_route_topk(1, 1, 1, 1, 4, 5000, 64, 3, 0.125, 1, None, None) == bad  # Np
    assert lib.sla2h_route_topk(1, 1, 1, 1, 4, 8, 64, 9, 0.125, 1, None, None) == bad     # T > Np
    # q, dq, kt(NULL), vt, q8, k8, qs, ks, kb, comp, alpha, alpha_stride, lut, dtype, B, H, L,
    # D, E, Np, T, scale, eps_l, flags, o, dout, stream: dq without the key operand tiles
    assert lib.sla2h_fwd_jvp(1, 1, None, 1, 1, 1, 1, 1, None, 1, 1, 1, 1, 1, 1, 1, 128, 64,
                             64, 2, 1, 0.125, 1e-5, 0, 1, 1, None) == bad
    assert lib.sla2h_linear_states(1, None, 1, None, 1, 1, 1, 100, 64, 64, 3, 1, None, 1, None,
                                   1, None, 1, None, 1, None, None) == bad  # Np > ceil(L/E)
    # tangent states without the key operand tiles
    assert lib.sla2h_linear_states(1, 1, 1, 1, 1, 1, 1, 128, 64, 64, 2, 1, 1, 1, 1,
                                   None, None, None, None, 1, None, None) == bad
    # training forward: q, k, v, dtype, B, H, L, D, E, q8, qs, k8, ks, v8f, vs, stream
    assert lib.sla2h_quant_train(1, 1, 1, 1, 1, 30000, 128, 64, 64, 1, 1, 1, 1, 1, 1, None) == bad
    assert lib.sla2h_quant_train(1, 1, None, 1, 1, 1, 128, 64, 64, 1, 1, 1, 1, 1, 1, None) == bad
    # q, q8, qs, k8, ks, v8f, vs, lut, dtype, B, H, L, D, E, Np, T, scale, o_s, lse, qphi
    assert lib.sla2h_sparse_fwd_qat(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 128, 64, 64, 2, 3, 0.125,
                                    1, 1, 1, None) == bad                   # T > Np
    assert lib.sla2h_sparse_fwd_qat(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 100000, 64, 64, 1, 1,
                                    0.125, 1, 1, 1, None) == bad            # tail > 1024 tiles
    assert lib.sla2h_linear_states_qat(1, 1, 1, 1, 1, 128, 64, 64, 1, 1, None, 1, None, None) == bad
    # the allocation-free complement: a 6 MiB bit-mask workspace (B=1, H=3, Mb=Np=4096) is
    # over its 4 MiB static array, rejected before any device call
    assert lib.sla2h_complement_workspace_bytes(1, 3, 4096, 4096) == 6 << 20
    assert lib.sla2h_complement_noalloc(1, None, 1, None, 1, 1, 3, 4096, 4096, 64, 1, 1,
                                        None) == bad
    # q, k, vt, lut, dtype, B, H, L, D, bq, bk, T, scale, o_s, lse, qphi: bq 96 unsupported
    assert lib.sla2h_sparse_fwd_1d(1, 1, 1, 1, 1, 1, 1, 640, 64, 96, 64, 2, 0.125, 1, 1, 1,
                                   None) == bad
    # qphi, comp, Hall, o_s, alpha, alpha_stride, dtype, B, H, L, D, E, eps, o, o_l, den
    assert lib.sla2h_linear_mix_qat(1, 1, 1, 1, 1, -1, 1, 1, 1, 128, 64, 64, 1e-5, 1, 1, 1,
                                    None) == bad


def test_ops_refuse_cpu_tensors():
    x = torch.zeros(1, 1, 64, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        ops.quantize(x)
    from imfvideo_amd.sla2_cube_qat import sla2_cube_qat_jvp_fused
    with pytest.raises(RuntimeError, match="GPU only"):
        sla2_cube_qat_jvp_fused(x, x, x, x, x, x, 0.9, 0.5, 1, 64, 0)


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(RuntimeError, match="build it"):
        _lib.load()


def test_no_alloc_capacity_at_the_29952_token_shape():
    """The static 4 MiB bit-mask array of sla2h_complement_noalloc covers B*H up to
    145 heads at Mb = Np = 468 (28,800 B each), the figure the header states."""
    lib = _lib.load()
    cap = 4 << 20
    assert lib.sla2h_complement_workspace_bytes(1, 1, 468, 468) == 28_800
    assert lib.sla2h_complement_workspace_bytes(1, 145, 468, 468) <= cap
    assert lib.sla2h_complement_workspace_bytes(1, 146, 468, 468) > cap
