"""Session-level operations of the read/keep path (the reference's
``maskahead.runtime.session``).

``value_score`` is the one scoring rule behind both decisions of the reference: the
selector feeds it the current block's mass, lookahead eviction the mass of the next
blocks (runtime/session.py:27-40).  Here it runs in the gfx950 kernels of
``ma_value_score``, with the reference's bf16 rounding points.

``evict_to`` is the session's eviction step (session.py:270-361): the eviction state's
compaction, then the lazy / full rebuild of a packed cache (ma_rebuild_plan,
ma_rebuild_packed) or the exact compaction of a 16-bit one.
"""

from __future__ import annotations

import torch

from ..kernels.keep import value_score as _value_score


def value_score(a: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """a_i * ||v_i - c||, c = sum_j a_j v_j / sum_j a_j.  a [..., n] f32, v [..., n, d]
    -> [..., n] f32 (session.py:27-40).  The environment variable BITSIEVE_VSCORE_FP32=1
    selects the f32 branch, as in the reference."""
    return _value_score(a, v)


def evict_to(cache, state, keep: torch.Tensor, cfg, *, next_position: int, phys_compact: bool = True,
             state_done: bool = False) -> None:
    """Keep live entries keep [L, B, Hkv, C]; then bring the physical cache in line
    (``BitSieveSession._evict_to``, session.py:270-361).

    cfg.compaction = "lazy" (packed caches): a key group that keeps at least
    ceil(repack_below * 32) of its entries is copied bit-exactly (its dead slots stay, to
    be masked); survivors of sparser groups and staged bf16 entries outside the recent
    window are quantized into fresh groups; the window and a stored-but-unadmitted
    prefill chunk stay as they are.  "full" re-quantizes every survivor; "none" (or
    phys_compact=False) only drops the entries from the state.  16-bit caches are
    compacted exactly.  ``next_position``: the first position not admitted yet (the
    session's _next_position).  The plan runs in ma_rebuild_plan, the data movement and
    the state's new slots in one ma_rebuild_packed launch; two host synchronisations
    (the plan's counts and the rebuild's status), as in the reference."""
    import math

    from ..kernels.rebuild import rebuild_plan

    if not state_done:
        state.compact(keep)
    mode = cfg.compaction if phys_compact else "none"
    if mode == "none":
        return
    dev = cache.device
    live = state.live
    tail = cache.get_seq_length() - next_position                 # stored, not admitted yet
    L, B, H = state.phys.shape[:3]
    tail_slots = torch.arange(cache.length - tail, cache.length, device=dev).view(1, 1, 1, -1).expand(L, B, H, tail)
    if not cache.quant.packed:
        phys = state.phys[..., :live].to(torch.int64)
        cache.compact(torch.cat([phys, tail_slots], -1))
        state.phys[..., :live] = torch.arange(live, device=dev, dtype=state.phys.dtype)
        return
    if mode not in ("lazy", "full"):
        raise ValueError(f"unknown eviction compaction: {mode}")
    gk, ql = cache.quant.key_token_group, cache.quantized_length
    ng = max(1, ql // gk)
    need = max(1, int(math.ceil(cfg.repack_below * gk))) if mode == "lazy" else gk + 1
    tail_groups = 0
    if tail and not cache.stage:                                   # the chunk: whole groups at the end
        if cache.residual_length or (cache.length - tail) % gk:
            raise RuntimeError("unadmitted tail must be whole key groups")
        tail_groups = tail // gk
    groups_before, enc_slots, stage_slots = rebuild_plan(
        state.phys, state.pos, live, quantized_length=ql, need=need, tail_groups=tail_groups,
        window=min(cfg.recent_window, live))
    empty = torch.empty((L, B, H, 0), dtype=torch.int64, device=dev)
    if tail and cache.stage:
        stage_slots = torch.cat([stage_slots, tail_slots], -1)
        groups_after = empty
    elif tail:
        groups_after = torch.arange(ng - tail_groups, ng, device=dev).expand(L, B, H, tail_groups)
    else:
        groups_after = empty
    cache._rebuild(groups_before, enc_slots, groups_after, stage_slots, phys=state.phys, live=live)
