"""Packed-cache eviction rebuild: host side of ``ma_rebuild_plan`` and ``ma_rebuild_packed``.

The reference computes the plan of a lazy / full compaction with torch ops on every
lane (runtime/session.py:288-345) and rebuilds the storage with per-layer gathers, a
dequantize of the whole layer and the append quantizers (cache.py:236-335).  Here one
kernel plans every lane at once and one launch moves every byte: group copies,
requantization, the bf16 stage, the slot remap and the eviction state's slots.
"""

from __future__ import annotations

import ctypes

import torch

from .. import _native as N

KG = 32


def _lanes2d(t: torch.Tensor, name: str) -> torch.Tensor:
    """[..., n] int64 index list -> [lanes, n] with contiguous rows: a view when the lanes
    are uniformly strided (a slice of a wider list, or one list broadcast to every lane,
    lane stride 0), else a copy."""
    if t.dtype != torch.int64:
        raise ValueError(f"{name} must be int64")
    lanes = 1
    for x in t.shape[:-1]:
        lanes *= int(x)
    t2 = t.reshape(lanes, t.shape[-1])
    if t2.shape[1] > 1 and t2.stride(1) != 1:
        t2 = t2.contiguous()
    return t2


def _stride(t2: torch.Tensor) -> int:
    """Lane stride of a [lanes, n] list (0 for a single lane or a broadcast list)."""
    return t2.stride(0) if t2.shape[0] > 1 else 0


def rebuild_plan(phys: torch.Tensor, pos: torch.Tensor, live: int, *, quantized_length: int, need: int,
                 tail_groups: int, window: int):
    """The lists of session.py:288-345 for the first ``live`` entries of every lane of the
    eviction state's phys int32 / pos [L, B, H, capacity] (after its compaction).

    Returns (groups_before, encode, stage) int64 [L, B, H, width], each cut to the largest
    count of any lane and padded with -1 -- the reference's ``packed`` lists.  One host
    synchronisation (the counts), as in the reference."""
    launched = rebuild_plan_launch(phys, pos, live, quantized_length=quantized_length, need=need,
                                   tail_groups=tail_groups, window=window)
    return rebuild_plan_cut(launched, launched[3].cpu())


def rebuild_plan_launch(phys: torch.Tensor, pos: torch.Tensor, live: int, *, quantized_length: int, need: int,
                        tail_groups: int, window: int):
    """rebuild_plan's launch alone, with no host synchronisation: (groups_before, encode,
    stage, counts, lead) with the lists at full width and counts int32 [lanes, 3] on the
    device.  rebuild_plan_cut finishes it from counts read back by the caller -- one read
    for the plans of several caches."""
    N.require_gpu(phys, "phys")
    if phys.dtype != torch.int32:
        raise ValueError("phys must be int32")
    if pos.dtype not in (torch.int32, torch.int64):
        raise ValueError("pos must be int32 or int64")
    lead = tuple(phys.shape[:-1])
    if tuple(pos.shape[:-1]) != lead or phys.shape[-1] < live or pos.shape[-1] < live:
        raise ValueError("phys and pos must be [..., capacity] with capacity >= live")
    p2 = phys.reshape(-1, phys.shape[-1])
    q2 = pos.reshape(-1, pos.shape[-1])
    if p2.stride(-1) != 1 or q2.stride(-1) != 1:
        raise ValueError("phys / pos rows must be contiguous")
    lanes = p2.shape[0]
    ng = max(1, quantized_length // KG)
    dev = phys.device
    gb = torch.empty((lanes, ng), device=dev, dtype=torch.int64)
    enc = torch.empty((lanes, max(live, 1)), device=dev, dtype=torch.int64)
    stg = torch.empty((lanes, max(live, 1)), device=dev, dtype=torch.int64)
    counts = torch.empty((lanes, 3), device=dev, dtype=torch.int32)
    if lanes:
        N.call("ma_rebuild_plan", p2.data_ptr(), p2.stride(0), q2.data_ptr(), int(pos.dtype == torch.int64),
               q2.stride(0), lanes, int(live), int(quantized_length), int(need), int(tail_groups), int(window),
               gb.data_ptr(), gb.stride(0), enc.data_ptr(), enc.stride(0), stg.data_ptr(), stg.stride(0),
               counts.data_ptr(), N.stream_of(phys))
    return gb, enc, stg, counts, lead


def rebuild_plan_cut(launched, counts_host: torch.Tensor):
    """The lists of a rebuild_plan_launch, cut to the largest count of any lane; counts_host
    is its counts tensor read back to the host."""
    gb, enc, stg, _, lead = launched
    flat = counts_host.reshape(-1).tolist()           # a few hundred ints: host lists, no tensor ops
    if not flat:
        empty = torch.empty((*lead, 0), device=gb.device, dtype=torch.int64)
        return empty, empty, empty
    if min(flat) < 0:
        raise N.KernelUnavailableError("rebuild plan: a lane holds more than 16384 live entries out of position "
                                       "order; only ordered lanes of that size are built")
    g1, m, st = max(flat[0::3]), max(flat[1::3]), max(flat[2::3])
    return (gb[:, :g1].reshape(*lead, g1), enc[:, :m].reshape(*lead, m), stg[:, :st].reshape(*lead, st))


def rebuild_packed(old, new, *, B: int, H: int, D: int, groups_before: torch.Tensor, encode: torch.Tensor,
                   groups_after: torch.Tensor, stage: torch.Tensor, remap: torch.Tensor,
                   phys: torch.Tensor | None = None, live: int = 0, check: bool = True) -> torch.Tensor | None:
    """One launch of ``ma_rebuild_packed``: old / new are Prefix objects (or their built
    MaPrefix descriptors) of the storage with layers folded into the batch axis (B =
    layers x batch); lists [lanes..., n]
    int64; remap int64 [lanes..., old length] written whole; phys (optional) int32
    [lanes..., capacity] rewritten in place for its first ``live`` entries.  Raises
    RuntimeError for a list entry outside the old storage (as the reference's gathers
    do) and AssertionError when a live entry maps to no new slot (session.py:354-355).
    check=False skips that read-back (a host synchronisation) and returns the per-lane
    status tensor instead, for raise_rebuild_status at a later synchronisation point."""
    lists = [_lanes2d(t, n) for t, n in ((groups_before, "groups_before"), (encode, "encode"),
                                         (groups_after, "groups_after"), (stage, "stage"))]
    lanes = B * H
    for t in lists:
        if t.shape[0] != lanes:
            raise ValueError(f"index lists must cover {lanes} lanes, got {t.shape[0]}")
    old_len = old.nq + old.nf
    r2 = remap.reshape(lanes, -1)
    if r2.shape[1] != old_len or r2.stride(-1) != 1 or remap.dtype != torch.int64:
        raise ValueError(f"remap must be int64 [lanes, {old_len}] with contiguous rows")
    dev = remap.device
    status = torch.empty((lanes,), device=dev, dtype=torch.int32)   # written for every lane
    ph_ptr, ph_stride = None, 0
    if phys is not None and live:
        p2 = phys.reshape(lanes, -1)
        if phys.dtype != torch.int32 or p2.stride(-1) != 1 or p2.shape[1] < live:
            raise ValueError("phys must be int32 [lanes, capacity >= live] with contiguous rows")
        ph_ptr, ph_stride = p2.data_ptr(), p2.stride(0)
    on = old if isinstance(old, N.MaPrefix) else old.native()
    nn = new if isinstance(new, N.MaPrefix) else new.native()
    gb, enc, ga, stg = lists
    N.call("ma_rebuild_packed", ctypes.byref(on), B, H, D, ctypes.byref(nn),
           gb.data_ptr(), _stride(gb), gb.shape[1], enc.data_ptr(), _stride(enc), enc.shape[1],
           ga.data_ptr(), _stride(ga), ga.shape[1], stg.data_ptr(), _stride(stg), stg.shape[1],
           r2.data_ptr(), r2.stride(0), ph_ptr, ph_stride, int(live if ph_ptr else 0), status.data_ptr(),
           N.stream_of(remap))
    if not check:
        return status
    raise_rebuild_status(status)
    return None


def raise_rebuild_status(status: torch.Tensor) -> None:
    """The errors of a rebuild from its per-lane status (one small copy to the host)."""
    s = int(status.cpu().max()) if status.numel() else 0   # no reduction kernel
    if s & 1:
        raise RuntimeError("rebuild: an index list names a slot or key group outside the cache")
    if s & 2:
        raise AssertionError("rebuild lost a live entry")
