"""Per-row selection kernels: the read-set top-k (session.py:1429-1438).

``topk_ascending`` replaces ``rank.masked_fill(dead, -inf).topk(k).indices.sort()``
with three kernel launches per call; ties at the k-th value go to the smaller index, so
the result is deterministic (torch.topk leaves that order unspecified).

The kernels keep each row's histogram in a state block that must be zero before its
first use and that every call leaves zero again.  One state buffer per (device, stream)
is kept here and grown (zero-filled) when a call has more rows: calls on one stream are
ordered, so they can share it, and a call on another stream (a selector side stream)
gets its own.  A caller may pass its own ``state`` instead.  The scratch workspace is
per call.
"""

from __future__ import annotations

import torch

from .. import _native as N
from .splitk import prefix_scores   # (splitk does not import this module)

_STATES: dict = {}
_MAX_STATES = 8


def _state(device: torch.device, nbytes: int, stream: int | None = None) -> torch.Tensor:
    """The zero-initialised select state of (`device`, its current stream -- `stream` when
    the caller has it), at least nbytes.  At most _MAX_STATES are kept (least recently
    used dropped first), so streams that come and go do not accumulate states; a state is
    only ever used on the stream it was allocated on, so dropping it hands the memory back
    to the caching allocator in that stream's order."""
    key = (device.index, stream if stream is not None else torch.cuda.current_stream(device).cuda_stream)
    st = _STATES.pop(key, None)
    if st is None or st.numel() < nbytes:
        # allocated and zero-filled on the current stream; the old one goes back to the
        # caching allocator, which reuses it in that stream's order
        st = torch.zeros((nbytes,), device=device, dtype=torch.uint8)
    _STATES[key] = st                              # most recently used last
    while len(_STATES) > _MAX_STATES:
        _STATES.pop(next(iter(_STATES)))
    return st


def topk_ascending(rank: torch.Tensor, k: int, mask: torch.Tensor | None = None, *,
                   out: torch.Tensor | None = None, values: torch.Tensor | None = None,
                   state: torch.Tensor | None = None) -> torch.Tensor:
    """rank [..., n] f32 on the GPU -> int64 [..., k] ascending indices of the k
    largest entries per row; mask (uint8/bool [..., n], 0 = dead) ranks an entry -inf.
    ``values`` (optional, f32 [..., k] contiguous) receives rank at those indices.
    ``state`` (optional, uint8, zero-filled before its first use, 256-byte aligned) replaces
    the device's shared select state."""
    N.require_gpu(rank, "rank")
    if rank.dtype != torch.float32:
        raise ValueError("rank must be float32")
    n = rank.shape[-1]
    k = int(k)
    if not 0 <= k <= n:
        raise ValueError(f"k={k} outside [0, {n}]")
    r2 = rank.reshape(-1, n)
    if r2.stride(-1) != 1:
        r2 = r2.contiguous()
    rows = r2.shape[0]
    m2 = None
    if mask is not None:
        m2 = mask.reshape(-1, n)
        if m2.dtype != torch.uint8:
            m2 = m2.to(torch.uint8)
        if m2.stride(-1) != 1:
            m2 = m2.contiguous()
    if out is None:
        out = torch.empty((*rank.shape[:-1], k), device=rank.device, dtype=torch.int64)
    if k == 0 or rows == 0:
        return out
    o2 = out.reshape(-1, k)
    if o2.stride(-1) != 1 or (rows > 1 and o2.data_ptr() != out.data_ptr()):
        raise ValueError("out must be a contiguous int64 [..., k] tensor")
    if values is not None and (not values.is_contiguous() or values.numel() != rows * k):
        raise ValueError("values must be a contiguous f32 [..., k] tensor")
    lib = N.load()
    ws_bytes = N.size_query("ma_topk_workspace_bytes", rows, n)
    if ws_bytes <= 0:
        raise N.KernelUnavailableError(f"ma_topk_select: n={n} exceeds the built maximum")
    stream = N.stream_of(rank)
    st = state if state is not None else _state(rank.device, N.size_query("ma_topk_state_bytes", rows), stream)
    ws = torch.empty((ws_bytes,), device=rank.device, dtype=torch.uint8)
    rc = lib.ma_topk_select(r2.data_ptr(), r2.stride(0) if rows > 1 else n, N.ptr(m2),
                            (m2.stride(0) if rows > 1 else n) if m2 is not None else 0, rows, n, k,
                            o2.data_ptr(), o2.stride(0) if rows > 1 else k, N.ptr(values), st.data_ptr(),
                            st.numel(), ws.data_ptr(), ws.numel(), stream)
    N.check(rc, "ma_topk_select")
    return out


def prefix_scores_topk(query, prefix, stats, q_rows, k: int, *, value: bool, rank: str = "score",
                       scaling=None, values: torch.Tensor | None = None):
    """prefix_scores followed by the read-set top-k over its mass (rank="mass") or score
    (rank="score", value-aware), masked by the prefix's mask, as session.py:1418-1438 runs
    them; the score pass builds the top-k's first-level histogram, so the pair costs one
    launch less than prefix_scores + topk_ascending and returns the same mass, score and
    indices.  Returns (mass, score, idx); idx int64 [B, Hkv, k] ascending."""
    if rank not in ("mass", "score") or (rank == "score" and not value):
        raise ValueError("rank must be 'mass', or 'score' with value=True")
    used = stats[3] if stats[3] is not None else prefix
    mp = stats[0]
    b, hkv, n = mp.shape[0], mp.shape[1], used.n
    k = int(k)
    if not 0 <= k <= n:
        raise ValueError(f"k={k} outside [0, {n}]")
    idx = torch.empty((b, hkv, k), device=query.device, dtype=torch.int64)
    if k == 0 or n == 0 or b * hkv == 0:
        mass, score = prefix_scores(query, prefix, stats, q_rows, value=value, scaling=scaling)
        return mass, score, idx
    rows = b * hkv
    if values is not None and (not values.is_contiguous() or values.numel() != rows * k):
        raise ValueError("values must be a contiguous f32 [B, Hkv, k] tensor")
    ws_bytes = N.size_query("ma_topk_workspace_bytes", rows, n)
    if ws_bytes <= 0:
        raise N.KernelUnavailableError(f"ma_topk_select: n={n} exceeds the built maximum")
    stream = N.stream_of(query)
    st = _state(query.device, N.size_query("ma_topk_state_bytes", rows), stream)
    code = 2 if rank == "score" else 1
    mass, score = prefix_scores(query, prefix, stats, q_rows, value=value, scaling=scaling, _topk_hist=(code, st))
    # mass / score are fresh contiguous [B, Hkv, n] f32; prefix_scores has checked the mask
    # (contiguous uint8 [B, Hkv, n])
    r = score if rank == "score" else mass
    ws = torch.empty((ws_bytes,), device=query.device, dtype=torch.uint8)
    rc = N.load().ma_topk_select_hist_ready(r.data_ptr(), n, N.ptr(used.mask), n if used.mask is not None else 0,
                                            rows, n, k, idx.data_ptr(), k, N.ptr(values), st.data_ptr(),
                                            st.numel(), ws.data_ptr(), ws.numel(), stream)
    N.check(rc, "ma_topk_select_hist_ready")
    return mass, score, idx
