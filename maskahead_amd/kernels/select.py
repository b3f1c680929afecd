"""Per-row selection kernels: the read-set top-k (session.py:1429-1438).

``topk_ascending`` replaces ``rank.masked_fill(dead, -inf).topk(k).indices.sort()``
with one kernel launch per call; ties at the k-th value go to the smaller index, so the
result is deterministic (torch.topk leaves that order unspecified).
"""

from __future__ import annotations

import torch

from .. import _native as N


def topk_ascending(rank: torch.Tensor, k: int, mask: torch.Tensor | None = None, *,
                   out: torch.Tensor | None = None, values: torch.Tensor | None = None) -> torch.Tensor:
    """rank [..., n] f32 on the GPU -> int64 [..., k] ascending indices of the k
    largest entries per row; mask (uint8/bool [..., n], 0 = dead) ranks an entry -inf.
    ``values`` (optional, f32 [..., k] contiguous) receives rank at those indices."""
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
    rc = lib.ma_topk_select(r2.data_ptr(), r2.stride(0) if rows > 1 else n, N.ptr(m2),
                            (m2.stride(0) if rows > 1 else n) if m2 is not None else 0, rows, n, k,
                            o2.data_ptr(), o2.stride(0) if rows > 1 else k, N.ptr(values), N.stream_of(rank))
    N.check(rc, "ma_topk_select")
    return out
