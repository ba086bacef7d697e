"""ctypes binding of the gfx950 C-ABI library ``libsla2hip.so``.

The library is loaded after ``torch`` so that its HIP runtime dependency
(``libamdhip64.so.7``) binds to the runtime torch already holds: device
pointers from torch's allocator and torch's streams are then valid inside
the library.  There is no fallback: a missing library raises.
"""

import ctypes
import os

import torch  # noqa: F401  (must be loaded first, see module docstring)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsla2hip.so")

_c_int, _c_i64, _c_f, _p = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/sla2h.h
SIGNATURES = {
    "sla2h_version": (_c_int, []),
    "sla2h_error_string": (ctypes.c_char_p, [_c_int]),
    "sla2h_quantize": (_c_int, [_p, _c_int, _c_i64, _c_i64, _c_int, _c_int, _p, _p, _p]),
    "sla2h_quant_pool_qk": (_c_int, [_p, _p, _c_int, _c_int, _c_int, _c_i64, _c_int, _c_int,
                                     _c_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p]),
    "sla2h_route_topk": (_c_int, [_p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                  _c_f, _p, _p, _p]),
    "sla2h_linear_states": (_c_int, [_p, _p, _p, _p, _c_int, _c_int, _c_int, _c_i64, _c_int,
                                     _c_int, _c_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                     _p]),
    "sla2h_complement_record_bytes": (ctypes.c_size_t, [_c_int]),
    "sla2h_complement_workspace_bytes": (ctypes.c_size_t, [_c_int, _c_int, _c_int, _c_int]),
    "sla2h_complement": (_c_int, [_p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int,
                                  _c_int, _p, _p, _p]),
    "sla2h_complement_noalloc": (_c_int, [_p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int,
                                          _c_int, _c_int, _p, _p]),
    "sla2h_fwd_jvp": (_c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _c_int, _p,
                               _c_int, _c_int, _c_int, _c_i64, _c_int, _c_int, _c_int, _c_int,
                               _c_f, _c_f, _c_int, _p, _p, _p]),
    "sla2h_pool_blocks": (_c_int, [_p, _c_int, _c_i64, _c_i64, _c_int, _c_int, _p, _c_int, _p,
                                   _p]),
    "sla2h_fwd_jvp_1d": (_c_int, [_p, _p, _p, _p, _p, _p, _c_int, _p, _c_int, _c_int, _c_int,
                                  _c_i64, _c_int, _c_int, _c_int, _c_int, _c_f, _c_f, _p, _p,
                                  _p]),
    "sla2h_rmsnorm_jvp": (_c_int, [_p, _p, _c_int, _p, _c_i64, _c_int, _c_i64, _p, _p, _c_i64,
                                   _c_int, _c_f, _p]),
    "sla2h_mla_qkv_prep": (_c_int, [_p, _p, _p, _c_i64, _p, _p, _p, _p, _p, _c_int, _c_int,
                                    _c_int, _c_int, _c_int, _c_int, _c_int, _c_f, _p, _p, _p, _p,
                                    _p, _p, _p]),
    "sla2h_mla_out_gate": (_c_int, [_p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _p,
                                    _p]),
    "sla2h_situ_jvp": (_c_int, [_p, _c_i64, _c_int, _c_f, _c_int, _p, _p]),
    "sla2h_rmsnorm_fwd": (_c_int, [_p, _c_int, _c_i64, _c_int, _c_i64, _p, _c_f, _p, _p]),
    "sla2h_rmsnorm_bwd_workspace_bytes": (ctypes.c_size_t, [_c_i64, _c_int]),
    "sla2h_gate_mul_fwd": (_c_int, [_p, _p, _c_int, _c_i64, _p, _p]),
    "sla2h_gate_mul_bwd": (_c_int, [_p, _p, _p, _c_int, _c_i64, _p, _p, _p]),
    "sla2h_attn_in_fwd": (_c_int, [_p, _c_int, _c_i64, _c_i64, _c_i64, _p, _c_int, _c_i64,
                                   _c_i64, _c_i64, _c_int, _c_int, _c_i64, _p, _p]),
    "sla2h_attn_in_bwd": (_c_int, [_p, _p, _c_int, _c_i64, _c_i64, _c_i64, _p, _c_int, _c_i64,
                                   _c_i64, _c_i64, _c_int, _c_int, _c_i64, _p]),
    "sla2h_attn_gate_fwd": (_c_int, [_p, _p, _c_int, _c_int, _c_int, _c_i64, _p, _p]),
    "sla2h_attn_gate_bwd": (_c_int, [_p, _p, _p, _c_int, _c_int, _c_int, _c_i64, _p, _p, _p]),
    "sla2h_rmsnorm_fwd16": (_c_int, [_p, _c_i64, _c_int, _c_i64, _p, _c_f, _c_int, _p, _p]),
    "sla2h_rmsnorm_bwd_sum": (_c_int, [_p, _c_i64, _c_int, _c_i64, _p, _p, _p, _p, _c_int, _p,
                                       _c_f, _p, _p, _p, _p]),
    "sla2h_rmsnorm_bwd": (_c_int, [_p, _c_int, _c_i64, _c_int, _c_i64, _p, _p, _c_f, _p, _p, _p,
                                   _p]),
    "sla2h_residual_scale_fwd": (_c_int, [_p, _p, _c_int, _p, _c_i64, _c_int, _p, _p]),
    "sla2h_residual_scale_bwd_workspace_bytes": (ctypes.c_size_t, [_c_i64, _c_int]),
    "sla2h_residual_scale_bwd": (_c_int, [_p, _p, _c_int, _p, _c_i64, _c_int, _p, _p, _p, _p]),
    "sla2h_rope": (_c_int, [_p, _c_int, _c_i64, _c_i64, _c_int, _c_int, _c_i64, _c_i64, _c_i64,
                            _p, _p, _c_int, _p, _p]),
    "sla2h_situ_mul_fwd": (_c_int, [_p, _p, _c_int, _c_i64, _c_int, _c_i64, _c_i64, _c_f, _c_f,
                                    _p, _p]),
    "sla2h_situ_mul_bwd": (_c_int, [_p, _p, _p, _c_int, _c_i64, _c_int, _c_i64, _c_i64, _c_f,
                                    _c_f, _p, _p, _p]),
    "sla2h_quant_train": (_c_int, [_p, _p, _p, _c_int, _c_int, _c_int, _c_i64, _c_int, _c_int,
                                   _p, _p, _p, _p, _p, _p, _p]),
    "sla2h_sparse_fwd_qat": (_c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int,
                                      _c_i64, _c_int, _c_int, _c_int, _c_int, _c_f, _p, _p, _p,
                                      _p]),
    "sla2h_linear_states_qat": (_c_int, [_p, _p, _c_int, _c_int, _c_int, _c_i64, _c_int, _c_int,
                                         _p, _p, _p, _p, _p, _p]),
    "sla2h_sparse_fwd_1d": (_c_int, [_p, _p, _p, _p, _c_int, _c_int, _c_int, _c_i64, _c_int,
                                     _c_int, _c_int, _c_int, _c_f, _p, _p, _p, _p]),
    "sla2h_linear_mix_qat": (_c_int, [_p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int,
                                      _c_i64, _c_int, _c_int, _c_f, _p, _p, _p, _p]),
    "sla2h_linear_mix_score": (_c_int, [_p, _p, _p, _p, _p, _p, _c_int, _p, _p, _c_int, _c_int,
                                        _c_int, _c_int, _c_i64, _c_int, _c_int, _c_f, _p, _p, _p,
                                        _p]),
    "sla2h_sla2_fused_workspace_bytes": (ctypes.c_size_t, [_c_int, _c_int, _c_i64, _c_int]),
    "sla2h_sla2_forward_fused": (_c_int, [_p, _p, _p, _p, _p, _c_int, _p, _p, _p, _p, _p, _p, _p,
                                          _p, _c_int, _p, _c_int, _c_int, _c_int, _c_int, _c_i64,
                                          _c_int, _c_int, _c_f, _c_f, _p, _p, _p]),
    "sla2h_quantize_v8f": (_c_int, [_p, _c_int, _c_i64, _c_i64, _c_int, _c_int, _p, _p, _p]),
    "sla2h_quantize_trunc": (_c_int, [_p, _c_int, _c_i64, _c_i64, _c_int, _c_int, _p, _p, _p]),
    "sla2h_sparse_fwd_int8": (_c_int, [_p, _p, _p, _c_int, _p, _p, _p, _p, _p, _c_int, _c_int,
                                       _c_int, _c_i64, _c_int, _c_int, _c_int, _c_f, _p, _p, _p,
                                       _p]),
    "sla2h_hblocks_states": (_c_int, [_p, _p, _c_int, _c_int, _c_int, _c_i64, _c_int, _c_int,
                                      _p, _p, _p, _p, _p, _p]),
    "sla2h_lin_fwd3": (_c_int, [_p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_i64, _c_int,
                                _c_int, _c_f, _p, _p]),
    "sla2h_bwd_prep": (_c_int, [_p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_i64,
                                _c_int, _c_int, _p, _p, _p, _p, _p, _p, _p, _p]),
    "sla2h_complement_bwd": (_c_int, [_p, _p, _p, _c_int, _c_int, _c_int, _c_int, _c_int, _p,
                                      _p, _p, _p]),
    "sla2h_bwd_dq": (_c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _c_int, _c_int,
                              _c_int, _c_i64, _c_int, _c_int, _c_int, _c_f, _p, _p]),
    "sla2h_bwd_dkdv": (_c_int, [_p, _p, _p, _p, _p, _p, _p, _p, _c_int, _c_int, _c_int, _c_i64,
                                _c_int, _c_int, _c_f, _p, _p, _p]),
}

_LIB = None


def load():
    """Return the loaded library, raising if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m imfvideo_amd.build` "
            "(there is no non-HIP implementation of these ops)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(code, what):
    """Raise RuntimeError for a nonzero hipError_t returned by `what`."""
    if code != 0:
        msg = load().sla2h_error_string(code)
        msg = msg.decode() if msg else "unknown error"
        raise RuntimeError(f"{what} failed: hipError {code} ({msg})")
