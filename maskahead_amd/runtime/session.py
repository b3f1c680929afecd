"""Session-level operations of the read/keep path (the reference's
``maskahead.runtime.session``).

``value_score`` is the one scoring rule behind both decisions of the reference: the
selector feeds it the current block's mass, lookahead eviction the mass of the next
blocks (runtime/session.py:27-40).  Here it runs in the gfx950 kernels of
``ma_value_score``, with the reference's bf16 rounding points.

``evict_to`` is the session's eviction step (session.py:270-361): the eviction state's
compaction, then the lazy / full rebuild of a packed cache (ma_rebuild_plan,
ma_rebuild_packed) or the exact compaction of a 16-bit one.  ``lookahead_evict``
(session.py:1985-2034) scores the live entries with the step-0 and probe masses and
evicts to the budget; ``live_slot_masks`` (session.py:240-255) gives the attention
kernels the live slots of a cache that keeps dead slots after a lazy rebuild.
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
             state_done: bool = False, check: bool = True) -> None:
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
    (the plan's counts and the rebuild's status), as in the reference.  check=False keeps
    only the first: the rebuild's status is read at the next rebuild (or
    cache.check_rebuild())."""
    pending = _evict_begin(cache, state, keep, cfg, next_position=next_position, phys_compact=phys_compact,
                           state_done=state_done)
    if pending is not None:
        _evict_finish(pending, pending.plan[3].cpu(), check=check)


class _PendingEviction:
    """An eviction whose plan is launched and whose counts are not read back yet."""

    __slots__ = ("cache", "state", "plan", "tail", "tail_slots", "tail_groups", "ng", "lead")

    def __init__(self, **kw):
        for k, v in kw.items():
            setattr(self, k, v)


def _evict_begin(cache, state, keep, cfg, *, next_position: int, phys_compact: bool = True,
                 state_done: bool = False):
    """evict_to up to the plan's launch (no host synchronisation): the state compacted and,
    for a packed cache, the rebuild plan enqueued -- returned for _evict_finish; None when
    the eviction is already complete (no physical compaction, or a 16-bit cache)."""
    import math

    from ..kernels.rebuild import rebuild_plan_launch

    if not state_done:
        state.compact(keep)
    mode = cfg.compaction if phys_compact else "none"
    if mode == "none":
        return None
    dev = cache.device
    live = state.live
    tail = cache.get_seq_length() - next_position                 # stored, not admitted yet
    L, B, H = state.phys.shape[:3]
    tail_slots = torch.arange(cache.length - tail, cache.length, device=dev).view(1, 1, 1, -1).expand(L, B, H, tail)
    if not cache.quant.packed:
        phys = state.phys[..., :live].to(torch.int64)
        cache.compact(torch.cat([phys, tail_slots], -1))
        state.phys[..., :live] = torch.arange(live, device=dev, dtype=state.phys.dtype)
        return None
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
    plan = rebuild_plan_launch(state.phys, state.pos, live, quantized_length=ql, need=need, tail_groups=tail_groups,
                               window=min(cfg.recent_window, live))
    return _PendingEviction(cache=cache, state=state, plan=plan, tail=tail, tail_slots=tail_slots,
                            tail_groups=tail_groups, ng=ng, lead=(L, B, H))


def _evict_finish(p, counts_host: torch.Tensor, *, check: bool = True) -> None:
    """The rest of evict_to once the plan's counts are on the host: the lists cut, the
    rebuild launched."""
    from ..kernels.rebuild import rebuild_plan_cut

    cache, state = p.cache, p.state
    L, B, H = p.lead
    groups_before, enc_slots, stage_slots = rebuild_plan_cut(p.plan, counts_host)
    dev = cache.device
    empty = torch.empty((L, B, H, 0), dtype=torch.int64, device=dev)
    if p.tail and cache.stage:
        stage_slots = torch.cat([stage_slots, p.tail_slots], -1)
        groups_after = empty
    elif p.tail:
        groups_after = torch.arange(p.ng - p.tail_groups, p.ng, device=dev).expand(L, B, H, p.tail_groups)
    else:
        groups_after = empty
    cache._rebuild(groups_before, enc_slots, groups_after, stage_slots, phys=state.phys, live=state.live,
                   check=check)


def live_slot_masks(cache, state) -> dict:
    """uint8 [B, Hkv, cache.length] per layer, 1 on the live slots (session.py:240-255);
    empty when every stored slot is live.  Pass it as FastLayerPath.slot_masks."""
    live = state.live
    if cache.length <= live:
        return {}
    phys = state.phys[..., :live].to(torch.int64)
    # the scatter below does not check its indices on the GPU: a slot outside the cache
    # (entries admitted with their positions as slots after a compaction, instead of
    # admit_new_entries) would write out of bounds -- refuse it here (one read-back)
    lo, hi = torch.stack(torch.aminmax(phys)).tolist() if live else (0, 0)
    if not 0 <= lo <= hi < cache.length:
        raise ValueError(f"eviction state holds slots outside the cache's {cache.length} (admit entries "
                         "appended after a compaction with admit_new_entries)")
    # every layer's mask in one [L, B, Hkv, length] tensor: three launches, not three per layer
    m = torch.zeros((state.num_layers, cache.batch_size, cache.num_kv_heads, cache.length), dtype=torch.uint8,
                    device=cache.device)
    m.scatter_(-1, phys, 1)
    return {layer: m[layer] for layer in range(state.num_layers)}


def admit_new_entries(cache, state, next_position: int) -> int:
    """Give the cache positions committed since next_position a slot in the live set
    (BitSieveSession._admit_new_entries, session.py:215-229): positions next_position ..
    length-1, their slots the newest physical slots of the cache (after a compaction the
    slots no longer equal the positions).  Returns the new next_position."""
    length = cache.get_seq_length()
    if length > next_position:
        m = length - next_position
        state.append(torch.arange(next_position, length, device=cache.device),
                     phys=torch.arange(cache.length - m, cache.length, device=cache.device))
    return max(length, next_position)


def live_values(cache, state, layer_idx: int) -> torch.Tensor:
    """Values of the live entries of one layer, [B, Hkv, live, D] in the compute dtype
    (session.py:263-268), gathered from the packed or 16-bit cache by ma_gather_kv."""
    from ..kernels.ops import gather_packed_kv

    slots = state.phys[layer_idx, ..., :state.live].to(torch.int64)
    _, v = gather_packed_kv(cache.layer_view(layer_idx), slots, dtype=cache.compute_dtype)
    return v


def lookahead_scores(cache, state, a1: dict, a_probe: dict | None = None, *, use_value: bool = True,
                     per_slot: bool = False) -> torch.Tensor:
    """score [L, B, Hkv, live] of the lookahead policy for layers on the fast path
    (session.py:1995-2025): a = the step-0 mass of the block's own queries (a1[layer],
    live order) + the probe mass of the next blocks (a_probe[layer], when probed); the
    score is value_score(a, v_live) (lookahead_score "value") or a itself ("mass").
    per_slot=True: a1[layer] is the mass per physical slot [B, Hkv, cache.length] (a
    step 0 run without live_slots), put in live order here for every layer in one gather
    -- the reference's _to_live (session.py:257-261), once instead of once per layer;
    a_probe stays in live order."""
    from ..kernels.keep import value_score_slots
    from ..kernels.splitk import Prefix

    L, B, H, live = state.num_layers, cache.batch_size, cache.num_kv_heads, state.live
    a_all = torch.stack([a1[layer] for layer in range(L)])
    if per_slot:
        a_all = a_all.gather(-1, state.phys[..., :live].to(torch.int64))
    if a_probe is not None:
        for layer in range(L):
            if layer in a_probe:
                a_all[layer] += a_probe[layer]
    if not use_value:
        return a_all
    # value_score(a, live_values(cache, state, layer)) of every layer in one call, the layers
    # folded into the batch axis, from the cache's codes directly (the same bits, no gathered
    # [B, Hkv, live, D] rows)
    score = torch.empty_like(a_all)
    value_score_slots(a_all.view(L * B, H, live), Prefix.from_view(cache.all_layers_view()),
                      state.phys[..., :live].reshape(L * B, H, live), dtype=cache.compute_dtype,
                      out=score.view(L * B, H, live))
    return score


def lookahead_evict(cache, state, cfg, capacity: int, a1: dict, a_probe: dict | None = None, *,
                    next_position: int, phys_compact: bool = True, check: bool = True, per_slot: bool = False):
    """Evict to `capacity` with the lookahead score (session.py:1985-2034): the survivors
    of the eviction state (ma_keep_select) under that score, then evict_to.  Returns the
    keep set, or None when the live set already fits.  check=False (a decode loop's hot
    path) skips the two error read-backs that cost a host synchronisation each -- the keep
    set's order check, whose positions the state keeps ascending by construction, and the
    rebuild's status, read at the next rebuild -- leaving the plan's count read-back as
    the eviction's only synchronisation.  per_slot: a1 holds masses per physical slot
    (lookahead_scores)."""
    if state.live <= capacity:
        return None
    score = lookahead_scores(cache, state, a1, a_probe, use_value=cfg.lookahead_score != "mass", per_slot=per_slot)
    keep = state.survivors(cfg, capacity, None, score, check=check)
    evict_to(cache, state, keep, cfg, next_position=next_position, phys_compact=phys_compact, check=check)
    return keep


def lookahead_evict_batch(batch, cfg, capacity: int, *, check: bool = False, per_slot: bool = False) -> list:
    """lookahead_evict for the sequences of a batch that each have their own cache and
    eviction state: batch = [(cache, state, a1, a_probe, next_position), ...].  The keep
    scores, keep sets, state compactions and rebuild plans of every sequence are enqueued
    first, the plans' counts come back in one host synchronisation for the whole batch
    (instead of one per sequence), then every rebuild is launched.  Returns the keep sets
    (None where the live set already fits).  check as in lookahead_evict (default False:
    no order-check or rebuild-status read-back); per_slot as in lookahead_scores."""
    keeps, pend = [], []
    for cache, state, a1, a_probe, next_position in batch:
        if state.live <= capacity:
            keeps.append(None)
            continue
        score = lookahead_scores(cache, state, a1, a_probe, use_value=cfg.lookahead_score != "mass",
                                 per_slot=per_slot)
        keep = state.survivors(cfg, capacity, None, score, check=check)
        keeps.append(keep)
        p = _evict_begin(cache, state, keep, cfg, next_position=next_position)
        if p is not None:
            pend.append(p)
    if pend:
        counts = torch.cat([p.plan[3].reshape(-1) for p in pend]).cpu()
        at = 0
        for p in pend:
            n = p.plan[3].numel()
            _evict_finish(p, counts[at:at + n], check=check)
            at += n
    return keeps
