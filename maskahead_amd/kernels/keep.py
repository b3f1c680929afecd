"""Keep-path kernel ops: keep-set selection, the value-aware keep score, in-place
compaction of survivors and the append of a finalized block.

Host side of the gfx950 kernels behind ``ma_keep_select``, ``ma_value_score``,
``ma_value_score_slots``, ``ma_compact_tokens`` and ``ma_append_tokens``.  They replace the torch ops the
reference runs on the keep path: ``EvictionState.survivors`` (eviction.py:325-409),
``value_score`` (runtime/session.py:27-40), the gathers of ``PackedKVCache.compact``
(cache.py:342-367), ``compact_tokens`` (cache.py:659-678) and ``EvictionState.compact``
(eviction.py:411-418), and the bf16 ``stage_layer`` copy (cache.py:423-547).
"""

from __future__ import annotations

import ctypes
import math
import os

import torch

from .. import _native as N
from .select import _state as select_state


def keep_select(pos: torch.Tensor, score: torch.Tensor, capacity: int, window: int, *, sink_tokens: int = 0,
                pin: tuple | None = None, check: bool = True) -> torch.Tensor:
    """Keep set per lane: the W = min(window, C) newest entries plus the top (C - W) of
    ``score`` among the others, sinks (pos < sink_tokens) and pinned positions ranking
    +inf; int64 [..., C] live-axis indices in position order.

    pos int32/int64 [..., n] must increase strictly along the last axis (the eviction
    state's order); score f32 [..., n].  pin = (lo, hi) with lo an int or a per-batch
    tensor broadcast over the rows' batch axis (eviction.py:239-243): pass lo already
    expanded to the leading shape of ``pos`` as a tensor, or an int.  check=True reads
    back the per-row order flag (one host sync) and raises ValueError if positions do
    not increase."""
    N.require_gpu(score, "score")
    if pos.shape != score.shape:
        raise ValueError(f"pos {tuple(pos.shape)} and score {tuple(score.shape)} differ")
    if pos.dtype not in (torch.int32, torch.int64):
        raise ValueError("pos must be int32 or int64")
    if score.dtype != torch.float32:
        raise ValueError("score must be float32")
    n = pos.shape[-1]
    capacity = int(capacity)
    if not 0 <= capacity <= n:
        raise ValueError(f"capacity {capacity} outside [0, {n}]")
    if window < 0:
        raise ValueError("window must be non-negative")
    p2 = pos.reshape(-1, n)
    s2 = score.reshape(-1, n)
    if p2.stride(-1) != 1:
        p2 = p2.contiguous()
    if s2.stride(-1) != 1:
        s2 = s2.contiguous()
    rows = p2.shape[0]
    out = torch.empty((*pos.shape[:-1], capacity), device=score.device, dtype=torch.int64)
    if rows == 0 or capacity == 0:
        return out
    status = torch.zeros((rows,), device=score.device, dtype=torch.int32)
    has_pin, lo_rows, lo, hi = 0, None, 0, 0
    if pin is not None:
        has_pin = 1
        lo, hi = pin
        hi = int(hi)
        if isinstance(lo, torch.Tensor):
            lo_rows = lo.to(device=score.device, dtype=torch.int64).expand(pos.shape[:-1]).reshape(-1).contiguous()
            lo = 0
        else:
            lo = int(lo)
    lib = N.load()
    ws_bytes = N.size_query("ma_topk_workspace_bytes", rows, n)
    if ws_bytes <= 0:
        raise N.KernelUnavailableError(f"ma_keep_select: n={n} exceeds the built maximum")
    st = select_state(score.device, N.size_query("ma_topk_state_bytes", rows))
    ws = torch.empty((ws_bytes,), device=score.device, dtype=torch.uint8)
    rc = lib.ma_keep_select(p2.data_ptr(), 1 if p2.dtype == torch.int64 else 0, p2.stride(0) if rows > 1 else n,
                            s2.data_ptr(), s2.stride(0) if rows > 1 else n, rows, n, capacity, int(window),
                            int(sink_tokens), N.ptr(lo_rows), lo, hi, has_pin, out.data_ptr(), capacity,
                            status.data_ptr(), st.data_ptr(), st.numel(), ws.data_ptr(), ws.numel(),
                            N.stream_of(score))
    N.check(rc, "ma_keep_select")
    if check and bool(status.any()):
        raise ValueError("keep_select: live positions must increase strictly along each lane")
    return out


def value_score(a: torch.Tensor, v: torch.Tensor, *, fp32: bool | None = None, out: torch.Tensor | None = None):
    """a_i * ||v_i - c||, c = sum_j a_j v_j / sum_j a_j (runtime/session.py:27-40).

    a f32 [..., H, n], v [..., H, n, D] (bf16/f16/f32, innermost dim contiguous, any
    strides on the others) -> f32 [..., H, n].  Default: the reference's bf16 arithmetic
    (w = bf16(a), every step rounded as its bf16 tensors compute it); fp32=True, or the
    environment variable BITSIEVE_VSCORE_FP32=1 as in the reference, selects the f32
    branch."""
    N.require_gpu(v, "v")
    if fp32 is None:
        fp32 = os.environ.get("BITSIEVE_VSCORE_FP32") == "1"
    if a.dtype != torch.float32:
        raise ValueError("a must be float32")
    if v.shape[:-1] != a.shape:
        raise ValueError(f"a {tuple(a.shape)} does not match v {tuple(v.shape)}")
    n, d = v.shape[-2], v.shape[-1]
    lead = v.shape[:-2]
    h = lead[-1] if lead else 1
    v4 = v.reshape(-1, h, n, d) if v.ndim != 4 else v
    if v4.stride(-1) != 1:
        v4 = v4.contiguous()
    b = v4.shape[0]
    a2 = a.reshape(-1, n)
    if a2.stride(-1) != 1:
        a2 = a2.contiguous()
    if out is None:
        out = torch.empty(a.shape, device=v.device, dtype=torch.float32)
    o2 = out.view(-1, n)
    if n == 0:
        return out
    lib = N.load()
    rows = b * h
    ws_bytes = int(lib.ma_value_score_workspace_bytes(rows, n, d))
    if ws_bytes < 0:
        raise N.KernelUnavailableError(f"value_score: head_dim {d} not built (<= 128, multiple of 8)")
    ws = torch.empty((ws_bytes,), device=v.device, dtype=torch.uint8)
    rc = lib.ma_value_score(a2.data_ptr(), a2.stride(0) if rows > 1 else n, N.t4(v4), b, h, n, d, 1 if fp32 else 0,
                            o2.data_ptr(), o2.stride(0) if rows > 1 else n, ws.data_ptr(), ws.numel(),
                            N.stream_of(v))
    N.check(rc, "ma_value_score")
    return out


def value_score_slots(a: torch.Tensor, prefix, slots: torch.Tensor, *, dtype: torch.dtype = torch.bfloat16,
                      fp32: bool | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """value_score(a, v) where v[b, h, j] is the value of cache slot slots[b, h, j] of lane
    (b, h) of the cache lanes `prefix` (a kernels.splitk.Prefix) describes, as
    gather_packed_kv(prefix, slots, dtype=dtype) returns it: the lookahead keep score over
    the live entries (runtime/session.py: value_score(a, live_values(...)),
    session.py:263-268, 1995-2025) computed from the packed codes or 16-bit rows directly,
    bit for bit the same, without the gathered [B, H, n, D] rows.

    a f32 [B, H, n]; slots int32 [B, H, >= n] (entries contiguous, lanes uniformly
    strided, e.g. the eviction state's phys[layer]); returns f32 [B, H, n]."""
    from .splitk import Prefix

    if not isinstance(prefix, Prefix):
        raise TypeError("prefix must be a kernels.splitk.Prefix")
    N.require_gpu(a, "a")
    if fp32 is None:
        fp32 = os.environ.get("BITSIEVE_VSCORE_FP32") == "1"
    if a.dtype != torch.float32 or a.dim() != 3:
        raise ValueError("a must be float32 [B, H, n]")
    if slots.dtype != torch.int32 or slots.dim() != 3 or tuple(slots.shape[:2]) != tuple(a.shape[:2]):
        raise ValueError("slots must be int32 [B, H, >= n] matching a")
    b, h, n = a.shape
    if slots.shape[2] < n:
        raise ValueError(f"slots hold {slots.shape[2]} entries per lane, {n} needed")
    s2 = slots[..., :n]
    if s2.stride(-1) != 1 or (b > 1 and s2.stride(0) != h * s2.stride(1)):
        s2 = s2.contiguous()
    sstride = s2.stride(1) if h > 1 else (s2.stride(0) if b > 1 else n)
    a2 = a if a.is_contiguous() else a.contiguous()
    if out is None:
        out = torch.empty((b, h, n), device=a.device, dtype=torch.float32)
    if n == 0:
        return out
    src = prefix.kq if prefix.nq else prefix.kf
    d = int(src.shape[-2] if prefix.nq else src.shape[-1])
    lib = N.load()
    ws_bytes = int(lib.ma_value_score_workspace_bytes(b * h, n, d))
    if ws_bytes < 0:
        raise N.KernelUnavailableError(f"value_score_slots: head_dim {d} not built")
    ws = torch.empty((ws_bytes,), device=a.device, dtype=torch.uint8)
    rc = lib.ma_value_score_slots(a2.data_ptr(), n, prefix.native(), s2.data_ptr(), sstride, b, h, n, d,
                                  N.dtype_code(dtype), 1 if fp32 else 0, out.data_ptr(), n, ws.data_ptr(), ws.numel(),
                                  N.stream_of(a))
    N.check(rc, "ma_value_score_slots")
    return out


def _rows_contiguous(shape, stride) -> bool:
    """Whether the dims (shape, stride) after the token axis form one contiguous row (dims
    of size 1 place no constraint)."""
    want = 1
    for size, st in zip(reversed(shape), reversed(stride)):
        if size != 1 and st != want:
            return False
        want *= size
    return True


def compact_tokens(planes, keep: torch.Tensor, n: int) -> None:
    """In place, for every lane (b, h) and i < C: row i of every plane becomes its old
    row keep[b, h, i].  planes: tensors [B, H, n_cap, ...] (token axis 2; everything
    after it is one row, contiguous); keep int64 [B, H, C]; n = rows in use (indices at
    or beyond n, or negative, give zero rows).  Up to 8 planes per launch pair; more are
    handled in groups."""
    if keep.ndim != 3:
        raise ValueError("keep must be [B, H, C]")
    N.require_gpu(keep, "keep")
    b, h, c = keep.shape
    if c > n:
        raise ValueError("compaction cannot grow the cache")
    k = keep if keep.dtype == torch.int64 else keep.to(torch.int64)
    if k.stride(-1) != 1:
        k = k.contiguous()
    lib = N.load()
    planes = [p for p in planes if p is not None]
    for i in range(0, len(planes), 8):
        group = planes[i:i + 8]
        bases, strides, rbytes = [], [], []
        for p in group:
            shp, std = p.shape, p.stride()
            if len(shp) < 3 or shp[0] != b or shp[1] != h or shp[2] < n:
                raise ValueError(f"plane of shape {tuple(shp)} does not fit keep {tuple(keep.shape)} / n={n}")
            if p.device != keep.device:
                raise ValueError("planes and keep must share a device")
            if not _rows_contiguous(shp[3:], std[3:]):
                raise ValueError("each token row of a plane must be contiguous")
            es = p.element_size()
            bases.append(p.data_ptr())
            strides += [std[0] * es, std[1] * es, std[2] * es]
            rbytes.append(math.prod(shp[3:]) * es)
        npl = len(group)
        base_arr = (ctypes.c_void_p * npl)(*bases)
        stride_arr = (ctypes.c_int64 * (3 * npl))(*strides)
        rb_arr = (ctypes.c_int32 * npl)(*rbytes)
        ws_bytes = int(lib.ma_compact_workspace_bytes(b * h, c, rb_arr, npl))
        ws = torch.empty((max(ws_bytes, 256),), device=keep.device, dtype=torch.uint8)
        rc = lib.ma_compact_tokens(base_arr, stride_arr, rb_arr, npl, b, h, int(n), k.data_ptr(),
                                   N.i64arr(k.stride(0), k.stride(1)), c, ws.data_ptr(), ws.numel(),
                                   N.stream_of(keep))
        N.check(rc, "ma_compact_tokens")


def append_tokens(src: torch.Tensor, dst: torch.Tensor, at: int) -> None:
    """dst[:, :, at:at+T] = src (converted to dst's dtype): [B, H, T, D] into the
    16-bit cache layout [B, H, capacity, D]."""
    N.require_gpu(dst, "dst")
    if src.ndim != 4 or dst.ndim != 4 or src.shape[:2] != dst.shape[:2] or src.shape[3] != dst.shape[3]:
        raise ValueError("append_tokens: src [B,H,T,D] and dst [B,H,cap,D] must agree on B, H, D")
    b, h, t, d = src.shape
    if at < 0 or at + t > dst.shape[2]:
        raise ValueError(f"append_tokens: [{at}, {at + t}) outside the capacity {dst.shape[2]}")
    lib = N.load()
    N.check(lib.ma_append_tokens(N.t4(src), N.t4(dst), b, h, t, d, int(at), N.stream_of(dst)), "ma_append_tokens")
