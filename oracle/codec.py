"""ctypes front end of oracle/codec.c -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Array arguments are numpy arrays (C-contiguous); torch callers pass ``.numpy()`` of
CPU tensors.  f16 / bf16 tensors travel as their uint16 bit patterns.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_SO = _HERE / "_build" / "liboracle_codec.so"
_lib = None


def build(force: bool = False) -> Path:
    """Compile codec.c with the committed Makefile (gcc only, no reference sources)."""
    if force or not _SO.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _SO


def lib():
    global _lib
    if _lib is None:
        build()
        _lib = ctypes.CDLL(str(_SO))
        _lib.oc_f16_to_f32.restype = ctypes.c_float
        _lib.oc_f16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.oc_f32_to_bf16.restype = ctypes.c_uint16
        _lib.oc_f32_to_bf16.argtypes = [ctypes.c_float]
        _lib.oc_bf16_to_f32.restype = ctypes.c_float
        _lib.oc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.oc_topk_ascending.restype = ctypes.c_int
        _lib.oc_keep_select.restype = ctypes.c_int
    return _lib


def _p(a: np.ndarray):
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("oracle arrays must be C-contiguous")
    return a.ctypes.data_as(ctypes.c_void_p)


def pack4(codes: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(codes.shape[:-1] + (codes.shape[-1] // 2,), dtype=np.uint8)
    lib().oc_pack4(_p(codes), ctypes.c_int64(codes.size), _p(out))
    return out


def unpack4(payload: np.ndarray) -> np.ndarray:
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    out = np.empty(payload.shape[:-1] + (payload.shape[-1] * 2,), dtype=np.uint8)
    lib().oc_unpack4(_p(payload), ctypes.c_int64(payload.size), _p(out))
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Element-wise RNE (scalar C routine; for small arrays and spot checks)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = lib().oc_f32_to_bf16
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.uint16).reshape(x.shape)


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    f = lib().oc_f16_to_f32
    return np.array([f(int(v)) for v in h.ravel()], dtype=np.float32).reshape(h.shape)


def dequant_keys4(payload: np.ndarray, scale: np.ndarray, zero: np.ndarray):
    """payload [..., G, D, KG/2] u8, scale/zero [..., G, D] (f16 bits as uint16 or
    float16) -> (f32 [..., G*KG, D], bf16 bits [..., G*KG, D])."""
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    scale = np.ascontiguousarray(scale).view(np.uint16)
    zero = np.ascontiguousarray(zero).view(np.uint16)
    *lead, g, d, half = payload.shape
    kg = half * 2
    rows = int(np.prod(lead)) if lead else 1
    p = payload.reshape(rows, g, d, half)
    s = scale.reshape(rows, g, d)
    z = zero.reshape(rows, g, d)
    o32 = np.empty((rows, g * kg, d), dtype=np.float32)
    o16 = np.empty((rows, g * kg, d), dtype=np.uint16)
    L = lib()
    for r in range(rows):
        pr, sr, zr = np.ascontiguousarray(p[r]), np.ascontiguousarray(s[r]), np.ascontiguousarray(z[r])
        o32r, o16r = o32[r], o16[r]
        L.oc_dequant_keys4(_p(pr), _p(sr), _p(zr), ctypes.c_int64(g), ctypes.c_int64(d),
                           ctypes.c_int64(kg), _p(o32r), _p(o16r))
    return o32.reshape(*lead, g * kg, d), o16.reshape(*lead, g * kg, d)


def dequant_values4(payload: np.ndarray, scale: np.ndarray, zero: np.ndarray):
    """payload [..., N, D/VG, VG/2] u8, scale/zero [..., N, D/VG] -> (f32, bf16 bits) [..., N, D]."""
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    scale = np.ascontiguousarray(scale).view(np.uint16)
    zero = np.ascontiguousarray(zero).view(np.uint16)
    *lead, n, ng, half = payload.shape
    vg = half * 2
    d = ng * vg
    rows = int(np.prod(lead)) if lead else 1
    p = payload.reshape(rows, n, ng, half)
    s = scale.reshape(rows, n, ng)
    z = zero.reshape(rows, n, ng)
    o32 = np.empty((rows, n, d), dtype=np.float32)
    o16 = np.empty((rows, n, d), dtype=np.uint16)
    L = lib()
    for r in range(rows):
        pr, sr, zr = np.ascontiguousarray(p[r]), np.ascontiguousarray(s[r]), np.ascontiguousarray(z[r])
        o32r, o16r = o32[r], o16[r]
        L.oc_dequant_values4(_p(pr), _p(sr), _p(zr), ctypes.c_int64(n), ctypes.c_int64(d),
                             ctypes.c_int64(vg), _p(o32r), _p(o16r))
    return o32.reshape(*lead, n, d), o16.reshape(*lead, n, d)


def topk_ascending(rank: np.ndarray, k: int, mask: np.ndarray | None = None) -> np.ndarray:
    """rank [..., n] f32 -> int64 [..., k]: the k largest per row (dead slots rank -inf,
    ties by ascending index), returned ascending (session.py:1429-1438)."""
    rank = np.ascontiguousarray(rank, dtype=np.float32)
    *lead, n = rank.shape
    rows = int(np.prod(lead)) if lead else 1
    r2 = rank.reshape(rows, n)
    m2 = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8).reshape(rows, n)
    out = np.empty((rows, k), dtype=np.int64)
    L = lib()
    for i in range(rows):
        ri = np.ascontiguousarray(r2[i])
        mi = None if m2 is None else np.ascontiguousarray(m2[i])
        oi = out[i]
        rc = L.oc_topk_ascending(_p(ri), None if mi is None else _p(mi), ctypes.c_int64(n),
                                 ctypes.c_int64(k), _p(oi))
        if rc:
            raise ValueError(f"oc_topk_ascending failed ({rc})")
    return out.reshape(*lead, k)


def keep_select(pos: np.ndarray, score: np.ndarray, capacity: int, window: int,
                sink_tokens: int = 0, pin: tuple[int, int] | None = None) -> np.ndarray:
    """pos int [..., n], score f32 [..., n] -> int64 [..., capacity] live-axis indices
    ordered by position (eviction.py:355-409)."""
    pos = np.ascontiguousarray(pos, dtype=np.int64)
    score = np.ascontiguousarray(score, dtype=np.float32)
    *lead, n = pos.shape
    rows = int(np.prod(lead)) if lead else 1
    p2, s2 = pos.reshape(rows, n), score.reshape(rows, n)
    out = np.empty((rows, capacity), dtype=np.int64)
    L = lib()
    lo, hi = pin if pin is not None else (0, 0)
    for i in range(rows):
        pi, si, oi = np.ascontiguousarray(p2[i]), np.ascontiguousarray(s2[i]), out[i]
        rc = L.oc_keep_select(_p(pi), _p(si), ctypes.c_int64(n), ctypes.c_int64(capacity),
                              ctypes.c_int64(window), ctypes.c_int64(sink_tokens),
                              ctypes.c_int(1 if pin is not None else 0), ctypes.c_int64(lo),
                              ctypes.c_int64(hi), _p(oi))
        if rc:
            raise ValueError(f"oc_keep_select failed ({rc})")
    return out.reshape(*lead, capacity)


def compact_rows(src: np.ndarray, keep: np.ndarray) -> np.ndarray:
    """src [..., n, *row], keep [..., c] -> [..., c, *row] (cache.py:342-367), out of place."""
    keep = np.ascontiguousarray(keep, dtype=np.int64)
    *lead, c = keep.shape
    rows = int(np.prod(lead)) if lead else 1
    n = src.shape[len(lead)]
    row_shape = src.shape[len(lead) + 1:]
    s2 = np.ascontiguousarray(src).reshape(rows, n, -1)
    row_bytes = s2.shape[-1] * s2.itemsize
    out = np.empty((rows, c, s2.shape[-1]), dtype=s2.dtype)
    k2 = keep.reshape(rows, c)
    L = lib()
    for i in range(rows):
        si, ki, oi = np.ascontiguousarray(s2[i]), np.ascontiguousarray(k2[i]), out[i]
        L.oc_compact_rows(_p(si), _p(ki), ctypes.c_int64(c), ctypes.c_int64(row_bytes), _p(oi))
    return out.reshape(*lead, c, *row_shape)
