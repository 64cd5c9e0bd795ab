"""ctypes loader for libm3x.so (the gfx950 kernels behind include/m3x.h).

torch is imported first so the library binds to the HIP runtime torch already loaded (both carry the soname
libamdhip64.so.7); device pointers and streams from torch are then valid inside the library.
There is no fallback: a missing or stale library raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see above)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libm3x.so")
ABI_VERSION = 16

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_long
_F = ctypes.c_float
_Z = ctypes.c_size_t

# name -> (restype, argtypes); the single source for the binding and for the export check in tests
SIGNATURES = {
    "m3x_version": (_I, []),
    "m3x_positions": (_I, [_P, _P, _P, _P, _I, _P]),
    "m3x_lengths_add": (_I, [_P, _P, _P, _I, _P]),
    "m3x_add_rms": (_I, [_P, _L, _P, _L, _P, _L, _P, _L, _P, _F, _I, _I, _P]),
    "m3x_linear_qk_rope": (_I, [_P, _L, _P, _F, _P, _P, _L, _P, _L, _L, _P, _P, _L, _L, _L, _P, _P, _P, _P, _L, _P, _P,
                                _F, _I, _I, _I, _I, _I, _I, _P]),
    "m3x_qk_norm_rope_cache": (_I, [_P, _L, _P, _L, _L, _P, _P, _L, _L, _L, _P, _P, _P, _P, _L, _P, _P, _F, _I, _I,
                                    _I, _I, _I, _P]),
    "m3x_decode_attn_workspace": (_Z, [_I, _I, _I, _I]),
    "m3x_decode_attn_item_bins": (_I, [_I, _I, _I, _I]),
    "m3x_decode_attn_items": (_L, [_P, _I, _I, _I, _I, _I, _P, _L]),
    "m3x_decode_attn": (_I, [_P, _L, _L, _P, _P, _L, _L, _L, _I, _P, _L, _L, _P, _P, _P, _F, _I, _I, _I, _I, _I, _I,
                             _P, _Z, _P]),
    "m3x_decode_attn_noalloc": (_I, [_P, _L, _L, _P, _P, _L, _L, _L, _I, _P, _L, _L, _P, _P, _P, _F, _I, _I, _I, _I,
                                     _I, _I, _P]),
    "m3x_packed_weight_elems": (_L, [_I, _I]),
    "m3x_pack_weight": (_I, [_P, _L, _I, _I, _P, _I, _P]),
    "m3x_linear": (_I, [_P, _L, _P, _P, _L, _I, _I, _I, _I, _P]),
    "m3x_linear_act": (_I, [_P, _L, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P]),
    "m3x_linear_resid": (_I, [_P, _L, _P, _P, _L, _P, _L, _I, _P, _L, _P, _I, _I, _I, _I, _I, _P]),
    "m3x_linear_normed": (_I, [_P, _L, _P, _P, _P, _F, _I, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P]),
    "m3x_act": (_I, [_P, _L, _P, _L, _I, _I, _I, _I, _P]),
    "m3x_add_norm": (_I, [_P, _L, _L, _P, _L, _L, _P, _L, _P, _P, _P, _P, _F, _I, _I, _I, _I, _I, _P]),
    "m3x_add_rows": (_I, [_P, _L, _P, _L, _P, _L, _I, _I, _I, _P]),
    "m3x_depth_attn": (_I, [_P, _L, _L, _P, _P, _P, _L, _L, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P]),
    "m3x_topk_sample": (_I, [_P, _L, _I, _P, _L, _F, _I, _I, _P, _L, _I, _I, _I, _P]),
    "m3x_topk_sample_embed": (_I, [_P, _L, _I, _P, _L, _F, _I, _I, _P, _L, _I, _I, _P, _L, _L, _P, _L, _P, _P, _P,
                                   _P, _F, _I, _I, _I, _P]),
    "m3x_cb0_sample": (_I, [_P, _L, _I, _I, _P, _P, _L, _P, _F, _P, _I, _P, _F, _P, _P, _P, _I, _P, _P, _P, _P, _P,
                            _P, _L, _P, _I, _P]),
    "m3x_philox_uniforms": (_I, [_P, _P, _P, _P, _L, _I, _I, _I, _P]),
    "m3x_philox_exponential": (_I, [_P, _P, _P, _L, _I, _I, _I, _P]),
    "m3x_philox_block": (_I, [_P, _P, _P, _P]),
    "m3x_ctr_add": (_I, [_P, _P, _I, _P]),
    "m3x_feedback": (_I, [_P, _P, _L, _P, _L, _P, _F, _F, _I, _I, _I, _I, _I, _P]),
    "m3x_copy_rows": (_I, [_P, _L, _P, _L, _L, _P, _L, _P, _I, _I, _I, _L, _P]),
    "m3x_cast_rows": (_I, [_P, _L, _I, _P, _L, _I, _I, _I, _P]),
    "m3x_code_ring_write": (_I, [_P, _L, _P, _P, _I, _I, _I, _I, _P]),
    "m3x_hist_push": (_I, [_P, _L, _P, _P, _P, _L, _I, _I, _P]),
    "m3x_loop_guard": (_I, [_P, _L, _P, _P, _P, _I, _I, _I, _I, ctypes.c_double, _I, _I, _P]),
    "m3x_tick_pack_width": (_I, [_I, _I, _I]),
    "m3x_tick_pack": (_I, [_P, _P, _P, _P, _L, _I, _P, _L, _I, _P, _L, _I, _P]),
    "m3x_depth_run_xchg_bytes": (_Z, []),
    "m3x_depth_run_args_bytes": (_Z, []),
    "m3x_depth_run": (_I, [_P, _P]),
    "m3x_depth_run_void": (_I, [_P, _P, _L, _I, _I, _I, _P]),
    "m3x_backbone_run_xchg_bytes": (_Z, []),
    "m3x_backbone_run_args_bytes": (_Z, []),
    "m3x_backbone_run_layer_bytes": (_Z, []),
    "m3x_backbone_run": (_I, [_P, _P]),
    "m3x_rvq_decode": (_I, [_P, _L, _P, _P, _L, _I, _I, _I, _I, _I, _P]),
    "m3x_dwconvt": (_I, [_P, _L, _P, _P, _L, _P, _P, _I, _I, _I, _I, _I, _P]),
    "m3x_conv_gather": (_I, [_P, _L, _P, _L, _P, _P, _L, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "m3x_rows_op": (_I, [_P, _L, _P, _P, _P, _L, _P, _L, _I, _I, _I, _I, _P]),
    "m3x_convt_overlap": (_I, [_P, _L, _P, _L, _P, _P, _P, _L, _I, _I, _I, _I, _I, _I, _I, _P]),
    "m3x_ring_attn": (_I, [_P, _L, _P, _P, _P, _P, _P, _P, _F, _P, _L, _I, _I, _I, _I, _I, _I, _I, _P]),
    "m3x_advance_tokens": (_I, [_P, _P, _I, _I, _I, _P]),
    "m3x_conv_gemm": (_I, [_P, _L, _P, _P, _P, _L, _P, _L, _I, _I, _I, _I, _P, _L, _P, _I, _I, _I, _I, _I, _P]),
    "m3x_resid_ln": (_I, [_P, _L, _P, _L, _P, _P, _P, _P, _L, _F, _I, _I, _I, _P]),
    "m3x_final_conv": (_I, [_P, _L, _P, _L, _P, _P, _F, _P, _L, _I, _I, _I, _I, _I, _I, _P]),
}

STATUS = {0: "ok", -1: "invalid argument", -2: "null pointer", -3: "workspace too small", -4: "launch failed",
          -5: "unsupported shape or dtype"}

_lib = None


def lib():
    """The loaded library (raises RuntimeError when it is missing, stale or incomplete)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"m3x native library not built: {LIB_PATH} is missing "
                           f"(build it with `make -C maya2-native_amd/csrc` or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        if not hasattr(L, name):
            raise RuntimeError(f"{LIB_PATH} does not export {name}: rebuild the library")
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    if L.m3x_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} has ABI version {L.m3x_version()}, expected {ABI_VERSION}: rebuild it")
    _lib = L
    return L


def check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed: {STATUS.get(status, status)} (status {status})")
