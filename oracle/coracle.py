"""ctypes binding of the C oracle (oracle/m3x_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg as the
checker; the product package never imports it. Build with `make -C oracle` (or __graft_entry__.build()).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libm3x_oracle.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_L = ctypes.c_long


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(_LIB_PATH)
        L.o_bf16_round.argtypes = [_F]
        L.o_bf16_round.restype = ctypes.c_uint16
        L.o_bf16_round_array.argtypes = [_P, _P, _L]
        L.o_expf.argtypes = [_F]
        L.o_expf.restype = _F
        L.o_expf_array.argtypes = [_P, _P, _L]
        L.o_add_rms.argtypes = [_P, _P, _P, _P, _P, _F, _I, _I]
        L.o_qk_norm_rope.argtypes = [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _F, _P, _P]
        L.o_topk_sample.argtypes = [_P, _I, _I, _F, _I]
        L.o_topk_sample.restype = _I
        L.o_topk_sample_many.argtypes = [_P, _I, _I, _P, _I, _P]
        L.o_topk_sample_rows.argtypes = [_P, _I, _I, _I, _F, _I, _P, _I, _P]
        L.o_cb0_sample.argtypes = [_P, _I, _I, _F, _I, _F, _F, _F, _P, _I, _P, ctypes.c_int64, _P, _P, _F, _P]
        L.o_cb0_sample.restype = _I
        L.o_philox4x32_10.argtypes = [_P, _P, _P]
        L.o_philox_uniform.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        L.o_philox_uniform.restype = _F
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round-to-nearest-even."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().o_bf16_round_array(_ptr(x), _ptr(y), x.size)
    return y


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().o_expf_array(_ptr(x), _ptr(y), x.size)
    return y


def add_rms(h: np.ndarray, a: np.ndarray | None, w: np.ndarray, eps: float):
    """h, a: uint16 bf16 [rows, n]; w: uint16 [n]. Returns (h_out or None, y) as uint16."""
    h = np.ascontiguousarray(h, np.uint16)
    rows, n = h.shape
    y = np.empty_like(h)
    ho = np.empty_like(h) if a is not None else None
    a = np.ascontiguousarray(a, np.uint16) if a is not None else None
    w = np.ascontiguousarray(w, np.uint16)
    lib().o_add_rms(_ptr(h), _ptr(a) if a is not None else None, _ptr(ho) if ho is not None else None, _ptr(y),
                    _ptr(w), eps, rows, n)
    return ho, y


def qk_norm_rope(qkv, H, KV, D, pos, cos, sin, wq, wk, eps):
    """qkv uint16 [rows, (H+2KV)*D]; pos int32 [rows]; cos/sin uint16 [cap, D]. Returns (q [rows,H,D], k [rows,KV,D])."""
    qkv = np.ascontiguousarray(qkv, np.uint16)
    rows = qkv.shape[0]
    pos = np.ascontiguousarray(pos, np.int32)
    cos = np.ascontiguousarray(cos, np.uint16)
    sin = np.ascontiguousarray(sin, np.uint16)
    wq = np.ascontiguousarray(wq, np.uint16)
    wk = np.ascontiguousarray(wk, np.uint16)
    q = np.empty((rows, H, D), np.uint16)
    k = np.empty((rows, KV, D), np.uint16)
    lib().o_qk_norm_rope(_ptr(qkv), rows, H, KV, D, _ptr(pos), _ptr(cos), _ptr(sin), _ptr(wq), _ptr(wk), eps,
                         _ptr(q), _ptr(k))
    return q, k


def topk_sample(x: np.ndarray, k: int, u: float, greedy: bool = False) -> int:
    """One transformed fp32 row."""
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().o_topk_sample(_ptr(x), x.size, k, u, int(greedy)))


def topk_sample_many(x: np.ndarray, k: int, u: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty(u.size, np.int32)
    lib().o_topk_sample_many(_ptr(x), x.size, k, _ptr(u), u.size, _ptr(out))
    return out


def topk_sample_rows(logits16: np.ndarray, inv_temp: float, k: int, u: np.ndarray | None, greedy=False,
                     is_f16=False) -> np.ndarray:
    logits16 = np.ascontiguousarray(logits16, np.uint16)
    B, V = logits16.shape
    uu = np.ascontiguousarray(u if u is not None else np.zeros(B), np.float32)
    out = np.empty(B, np.int32)
    lib().o_topk_sample_rows(_ptr(logits16), B, V, int(is_f16), inv_temp, k, _ptr(uu), int(greedy), _ptr(out))
    return out


def cb0_sample(logits16: np.ndarray, aeos: int, temp: float, k: int, bias: float, rep: float,
               hist: np.ndarray | None, frames: np.ndarray | None, min_frames: int, hazard: np.ndarray | None,
               ctr: np.ndarray | None, u: float, top_p: float = 1.0):
    """One seat. hist int64 [W] / frames int64 [1] / hazard float32 [1] / ctr int32 [1] are updated in place."""
    logits16 = np.ascontiguousarray(logits16, np.uint16)
    stop = np.zeros(1, np.int64)
    cb0 = lib().o_cb0_sample(_ptr(logits16), logits16.size, aeos, temp, k, top_p, bias, rep,
                             _ptr(hist) if hist is not None else None, 0 if hist is None else hist.size,
                             _ptr(frames) if frames is not None else None, min_frames,
                             _ptr(hazard) if hazard is not None else None, _ptr(ctr) if ctr is not None else None,
                             u, _ptr(stop))
    return int(cb0), int(stop[0])


def philox4x32_10(ctr, key) -> list[int]:
    c = np.asarray(ctr, np.uint32)
    k = np.asarray(key, np.uint32)
    o = np.empty(4, np.uint32)
    lib().o_philox4x32_10(_ptr(c), _ptr(k), _ptr(o))
    return [int(v) for v in o]


def philox_uniform(seed: int, ctr: int, level: int) -> float:
    return float(lib().o_philox_uniform(seed & 0xFFFFFFFF, ctr & 0xFFFFFFFF, level & 0xFFFFFFFF))
