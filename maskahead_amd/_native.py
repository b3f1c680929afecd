"""ctypes binding of libmaskahead_hip.so (the C ABI declared in include/maskahead_hip.h).

The library is built in-tree (maskahead_amd/libmaskahead_hip.so) by
``maskahead_amd.build.build()``.  There is no fallback: if the library is missing or a
kernel is not built for the requested shape, the call raises.
"""

from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path

import torch

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libmaskahead_hip.so"

MA_OK, MA_EINVAL, MA_EUNSUPPORTED, MA_EHIP, MA_EWORKSPACE = 0, -1, -2, -3, -4
MA_F32, MA_F16, MA_BF16 = 0, 1, 2

_DTYPE_CODE = {torch.float32: MA_F32, torch.float16: MA_F16, torch.bfloat16: MA_BF16}


class KernelUnavailableError(RuntimeError):
    """A requested kernel is not available: library missing, no GPU, or a shape / bit
    width / backend this build does not implement (the reference's ops.py:19-20)."""


class MaPrefix(ctypes.Structure):
    _fields_ = [
        ("kq", ctypes.c_void_p), ("ks", ctypes.c_void_p), ("kz", ctypes.c_void_p),
        ("vq", ctypes.c_void_p), ("vs", ctypes.c_void_p), ("vz", ctypes.c_void_p),
        ("kf", ctypes.c_void_p), ("vf", ctypes.c_void_p), ("mask", ctypes.c_void_p),
        ("skq", ctypes.c_int64 * 4), ("sks", ctypes.c_int64 * 3), ("svq", ctypes.c_int64 * 4),
        ("svs", ctypes.c_int64 * 3), ("skf", ctypes.c_int64 * 3), ("svf", ctypes.c_int64 * 3),
        ("nq", ctypes.c_int32), ("nf", ctypes.c_int32), ("kbits", ctypes.c_int32),
        ("vbits", ctypes.c_int32), ("kgroup", ctypes.c_int32), ("vgroup", ctypes.c_int32),
        ("fdtype", ctypes.c_int32), ("reserved", ctypes.c_int32),
    ]


class MaTensor4(ctypes.Structure):
    _fields_ = [("ptr", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("s", ctypes.c_int64 * 3)]


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_PREF = ctypes.POINTER(MaPrefix)
_T4 = MaTensor4
_I64P = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); must match include/maskahead_hip.h
SIGNATURES = {
    "ma_last_error": (ctypes.c_char_p, []),
    "ma_version": (_I, []),
    "ma_dequant_prefix": (_I, [_PREF, _I, _I, _I, _T4, _T4, _P]),
    "ma_splitk_workspace_bytes": (_I64, [_I, _I, _I, _I, _I, _I, _I, _I]),
    "ma_splitk_attention": (_I, [_T4, _I, _I, _I, _I, _PREF, _I, _T4, _T4, _I, _I, _I, _I, _F, _T4,
                                 _P, _P, _P, _I, _P, _I64, _P]),
    "ma_splitk_partial": (_I, [_T4, _I, _I, _I, _I, _PREF, _I, _T4, _T4, _I, _I, _I, _I, _F, _I, _P, _I64, _P]),
    "ma_splitk_merge": (_I, [_T4, _I, _I, _I, _I, _PREF, _I, _T4, _T4, _I, _I, _I, _I, _F, _T4, _P, _P, _P, _I, _P,
                             _I64, _P]),
    "ma_splitk_noalloc_max_bytes": (_I64, []),
    "ma_splitk_attention_noalloc": (_I, [_T4, _I, _I, _I, _I, _PREF, _I, _T4, _T4, _I, _I, _I, _I, _F, _T4,
                                         _P, _P, _P, _I, _P]),
    "ma_value_centre": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _I, _P, _P]),
    "ma_prefix_scores": (_I, [_T4, _I, _I, _I, _I, _PREF, _I, _P, _I, _P, _P, _P, _I, _F, _I, _I, _P,
                              _P, _P]),
    "ma_prefix_scores_path": (_I, [_I]),
    "ma_prefix_scores_hist": (_I, [_T4, _I, _I, _I, _I, _PREF, _I, _P, _I, _P, _P, _P, _I, _F, _I, _I, _P,
                                   _P, _I, _P, _I64, _P]),
    "ma_step0_workspace_bytes": (_I64, [_I, _I, _I, _I, _I, _I, _I]),
    "ma_step0": (_I, [_T4, _I, _I, _I, _I, _PREF, _I, _T4, _T4, _I, _F, _T4, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P,
                      _I, _P, _T4, _T4, _P, _I64, _P, _I64, _P]),
    "ma_keep_select": (_I, [_P, _I, _I64, _P, _I64, _I, _I, _I, _I, _I64, _P, _I64, _I64, _I, _P, _I64, _P,
                            _P, _I64, _P, _I64, _P]),
    "ma_value_score_workspace_bytes": (_I64, [_I, _I, _I]),
    "ma_value_score": (_I, [_P, _I64, _T4, _I, _I, _I, _I, _I, _P, _I64, _P, _I64, _P]),
    "ma_value_score_slots": (_I, [_P, _I64, _PREF, _P, _I64, _I, _I, _I, _I, _I, _I, _P, _I64, _P, _I64, _P]),
    "ma_compact_workspace_bytes": (_I64, [_I, _I, _P, _I]),
    "ma_compact_tokens": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _I64P, _I, _P, _I64, _P]),
    "ma_append_tokens": (_I, [_T4, _T4, _I, _I, _I, _I, _I, _P]),
    "ma_topk_state_bytes": (_I64, [_I]),
    "ma_topk_workspace_bytes": (_I64, [_I, _I]),
    "ma_topk_select": (_I, [_P, _I64, _P, _I64, _I, _I, _I, _P, _I64, _P, _P, _I64, _P, _I64, _P]),
    "ma_topk_select_hist_ready": (_I, [_P, _I64, _P, _I64, _I, _I, _I, _P, _I64, _P, _P, _I64, _P, _I64, _P]),
    "ma_gather_kv": (_I, [_PREF, _I, _I, _I, _P, _I64P, _I, _T4, _T4, _P]),
    "ma_quantize_keys": (_I, [_T4, _I, _I, _I, _I, _I, _P, _I64P, _P, _P, _I64P, _P]),
    "ma_quantize_values": (_I, [_T4, _I, _I, _I, _I, _I, _P, _I64P, _P, _P, _I64P, _P]),
    "ma_append_packed": (_I, [_T4, _T4, _I, _T4, _T4, _I, _I, _I, _I, _I, _I, _P, _I64P, _P, _P, _I64P, _P, _I64P,
                              _P, _P, _I64P, _P]),
    "ma_rebuild_plan": (_I, [_P, _I64, _P, _I, _I64, _I, _I, _I, _I, _I, _I, _P, _I64, _P, _I64, _P, _I64, _P, _P]),
    "ma_rebuild_packed": (_I, [_PREF, _I, _I, _I, _PREF, _P, _I64, _I, _P, _I64, _I, _P, _I64, _I, _P, _I64, _I,
                               _P, _I64, _P, _I64, _I, _P, _P]),
}

_lib = None


def load(path: Path | str | None = None):
    """Load (once) and return the ctypes library; raises KernelUnavailableError."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else Path(os.environ.get("MASKAHEAD_HIP_LIB", LIB_PATH))
    if not p.exists():
        raise KernelUnavailableError(
            f"{p} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(hipcc, gfx950) first")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


@functools.lru_cache(maxsize=4096)
def size_query(name: str, *args) -> int:
    """A workspace / state size entry point of the library (a pure function of its integer
    arguments and of the device's CU count), memoized: the host path calls them on every
    kernel call."""
    return int(getattr(load(), name)(*args))


def check(rc: int, what: str) -> None:
    if rc == MA_OK:
        return
    msg = load().ma_last_error().decode(errors="replace") or what
    if rc in (MA_EINVAL, MA_EWORKSPACE):
        raise ValueError(msg)
    if rc == MA_EUNSUPPORTED:
        raise KernelUnavailableError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    """Call entry point `name` of the library; a negative status raises (check)."""
    check(getattr(load(), name)(*args), name)


def require_gpu(t: torch.Tensor, name: str = "tensor") -> None:
    if not t.is_cuda:
        raise KernelUnavailableError(
            f"{name} is on {t.device}; the MI355X kernels need GPU tensors (the CPU path is "
            "the test oracle, not part of this package)")


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt}") from None


def stream_of(t: torch.Tensor) -> int:
    """The raw handle of the current stream of t's device (what torch's own kernels are
    launched on), without building a torch.cuda.Stream object."""
    return torch._C._cuda_getCurrentRawStream(t.get_device())


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def t4(t: torch.Tensor | None) -> MaTensor4:
    """[B, H, T, D] tensor with contiguous last dim -> MaTensor4 (strides b, h, t)."""
    m = MaTensor4()
    if t is None:
        return m
    s = t.stride()
    if len(s) != 4:
        raise ValueError(f"expected a 4-d tensor, got shape {tuple(t.shape)}")
    if s[3] != 1 and t.shape[3] > 1:
        raise ValueError("the innermost dimension must be contiguous")
    m.ptr = t.data_ptr()
    m.dtype = dtype_code(t.dtype)
    m.s[0], m.s[1], m.s[2] = s[0], s[1], s[2]
    return m


def i64arr(*vals) -> ctypes.Array:
    a = (ctypes.c_int64 * len(vals))()
    for i, v in enumerate(vals):
        a[i] = int(v)
    return a
