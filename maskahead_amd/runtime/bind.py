"""Delegation of a reference session's fast path to this package, in one call.

``bind_session(session)`` takes a ``BitSieveSession`` (runtime/session.py:97) -- or any
object with the same attributes -- and replaces, on that instance only, the methods
whose bodies run the read/keep path in torch:

  * ``_fast_step0`` (session.py:1403-1454): split-K attention, prefix statistics, mass and
    value-aware score, ``rank.topk().sort()`` and the gather -> one ``ma_step0`` call into
    the session's own compact buffers (``_ensure_state``), with the same side effects on
    the session (``_la_a1``, the EMA observation, the state's indices, the trace record);
  * ``_compact_attention`` (session.py:1286-1336): the block copy and SDPA over
    [selected | block] -> split-K over the compact buffer and the block's own tensors;
  * ``_fast_attend`` / ``_current_only`` / ``_prefix`` (session.py:1362-1401): probes and
    prefill chunks, with the prefix descriptor kept per layer;
  * ``_live_values`` (session.py:263-268): the live rows gathered by ``ma_gather_kv``
    instead of dequantizing the whole layer first;
  * when the session's cache is this package's ``PackedKVCache``: ``_evict_to``
    (session.py:270-361, planned and moved by ``ma_rebuild_plan`` / ``ma_rebuild_packed``)
    and ``_lookahead_evict`` (session.py:1985-2034, the keep score of every layer from
    the cache's codes by ``ma_value_score_slots``);
  * when the session's eviction state is still empty: the state itself, replaced by this
    package's ``EvictionState`` (``survivors`` by ``ma_keep_select``, ``compact`` by
    ``ma_compact_tokens``, eviction.py:325-418).

``bind_value_score(module)`` points a module's ``value_score`` (session.py:27-40, called
by the lookahead and EMA policies) at the HIP one.  Everything else in the session (the
generator hooks, the routing in ``_attend_main``, the policies' bookkeeping) stays the
reference's own code.
"""

from __future__ import annotations

import sys

from .._native import KernelUnavailableError
from ..kernels.step0 import Step0Buffers, step0_select
from .fastpath import FastLayerPath, fast_path_supported

_EMA_POLICIES = ("ema_recent", "ema_recent_value")


def _is_own_cache(cache) -> bool:
    from ..cache import PackedKVCache

    return isinstance(cache, PackedKVCache)


def bind_value_score(module):
    """Replace ``module.value_score`` (the reference session module's bf16 keep score,
    session.py:27-40) by this package's; returns the function it replaced."""
    from .session import value_score

    old = getattr(module, "value_score", None)
    module.value_score = value_score
    return old


def bind_session(session) -> FastLayerPath:
    """Route `session`'s fast-path methods through this package (see the module
    docstring).  Raises KernelUnavailableError, leaving the session untouched, when the
    session's configuration is one this library does not serve (fast_path_supported:
    the reference's own conditions plus the built bit widths, groups and head sizes).
    Call it after constructing the session and before its first forward.  Returns the
    FastLayerPath the bound methods share (its ``states`` is the session's own dict)."""
    s = session
    cfg = s.config
    ok, why = fast_path_supported(cfg, s.head_dim, s.cache.device.type)
    if not ok:
        raise KernelUnavailableError(f"the session's configuration is not served by the HIP path ({why})")
    fp = FastLayerPath(cache=s.cache, block_size=cfg.generation.block_size, value_aware=cfg.selector.value_aware,
                       sort_indices=cfg.selector.sort_indices, compute_dtype=s.compute_dtype,
                       dense_prefix_layers=cfg.selector.dense_prefix_layers, semantic=cfg.semantic)
    fp.states = s._states
    scale = s.head_dim ** -0.5
    step0_bufs: dict = {}
    step0_ws = Step0Buffers()
    record = getattr(sys.modules.get(type(s).__module__), "SelectionRecord", None)

    if s._eviction is not None and s._eviction.live == 0:
        from ..eviction import EvictionState

        if not isinstance(s._eviction, EvictionState):
            old = s._eviction
            s._eviction = EvictionState(num_layers=old.num_layers, batch_size=old.batch_size,
                                        num_kv_heads=old.num_kv_heads, capacity=cfg.eviction.capacity_floor,
                                        device=old.device, max_position=cfg.max_cache_tokens)

    def _prefix(layer_idx):
        # session.py:1362-1367: the layer's view with its live mask, the descriptor kept
        # while the cache's planes, lengths and the mask object are unchanged
        mask = s._slot_mask(layer_idx)
        if mask is None:
            fp.slot_masks.pop(layer_idx, None)
        else:
            fp.slot_masks[layer_idx] = mask
        return fp.prefix(layer_idx)

    def _current_only(query, current_key, current_value, causal, q_pos0):
        return fp.current_only(query, current_key, current_value, causal, q_pos0)

    def _fast_attend(layer_idx, query, current_key, current_value, *, causal=0, q_pos0=0, mass_rows=None):
        _prefix(layer_idx)
        return fp.attend(layer_idx, query, current_key, current_value, causal=causal, q_pos0=q_pos0,
                         mass_rows=mass_rows)

    def _fast_step0(layer_idx, query, current_key, current_value, dense):
        ev = s._eviction
        need_sel = not dense and cfg.semantic == "A" and bool(s.query_indices)
        need_mass = bool(s.query_indices) and ev is not None and ev.live > 0 and (
            s._la_pending is not None or cfg.eviction.policy in _EMA_POLICIES)
        prefix = _prefix(layer_idx)
        if prefix.n == 0:
            return fp.current_only(query, current_key, current_value, 0, 0)
        if not (need_sel or need_mass):
            return fp.step0(layer_idx, query, current_key, current_value, select=False, topk=0)
        if need_sel:
            rows = fp.rows(s.query_indices)
            k = s._effective_budget()
            state = s._ensure_state(layer_idx, k)
            bufs = step0_bufs.setdefault(layer_idx, Step0Buffers())
            out, _, mass, _, idx = step0_select(bufs, query, prefix, current_key, current_value, rows, k,
                                                value=cfg.selector.value_aware, scaling=scale,
                                                out_key=state.key[:, :, :k, :], out_value=state.value[:, :, :k, :],
                                                workspace=step0_ws)
        else:
            fp.query_indices = list(s.query_indices)
            out = fp.step0(layer_idx, query, current_key, current_value, select=False, topk=0, want_mass=True)
            mass = fp.last_mass.pop(layer_idx)
        if ev is not None:
            live_mass = s._to_live(layer_idx, mass)
            if s._la_pending is not None:
                s._la_a1[layer_idx] = live_mass if live_mass is not mass else mass.clone()
            if cfg.eviction.policy in _EMA_POLICIES:
                ev.observe(layer_idx, live_mass, cfg.eviction.decay, len(s.query_indices))
        if need_sel:
            # idx is this layer's reused step-0 buffer: valid until the layer's next step 0,
            # which replaces the state's read set anyway
            state.indices = idx
            state.selected_k = k
            if record is not None:
                s.trace.selections.append(record(
                    block=s.block_index, layer=layer_idx, old_cache_len=s.old_cache_len, selected_k=k,
                    selector_queries=s.query_indices, semantic=cfg.semantic, index_checksum=0))
        return out

    def _compact_attention(layer_idx, query, current_key, current_value):
        with s.timer.region("compact_attention", tensor=query, layer=layer_idx, block=s.block_index,
                            step=s.step_index):
            return fp.compact_attention(layer_idx, query, current_key, current_value)

    def _live_values(layer_idx):
        from .session import live_values

        return live_values(s.cache, s._eviction, layer_idx)

    s._prefix = _prefix
    s._current_only = _current_only
    s._fast_attend = _fast_attend
    s._fast_step0 = _fast_step0
    s._compact_attention = _compact_attention
    s._live_values = _live_values

    if _is_own_cache(s.cache):
        from ..eviction import EvictionState
        from .session import evict_to, lookahead_scores

        original_lookahead = s._lookahead_evict

        def _evict_to(keep, *, state_done=False):
            if s._attn_log is not None:
                s._log_eviction(keep, state_done)
            s._mask_epoch = getattr(s, "_mask_epoch", 0) + 1
            evict_to(s.cache, s._eviction, keep, cfg.eviction, next_position=s._next_position,
                     phys_compact=s._phys_compact, state_done=state_done)

        def _lookahead_evict(capacity):
            st = s._eviction
            if st.live <= capacity:
                return
            if not isinstance(st, EvictionState) or any(layer not in s._la_a1 for layer in range(st.num_layers)):
                return original_lookahead(capacity)      # layers scored on the reference's old path
            score = lookahead_scores(s.cache, st, s._la_a1, s._la_aprobe,
                                     use_value=cfg.eviction.lookahead_score != "mass")
            s._log_score(score, "lookahead_m1" if cfg.eviction.horizon_blocks == 1 else "lookahead", capacity)
            s._log_pairwise_eviction(capacity)
            if cfg.eviction.record_only:
                return
            before = st.live
            keep = st.survivors(cfg.eviction, capacity, None, score)
            s._evict_to(keep)
            s.trace.add_counter("evictions", 1)
            s.trace.add_counter("entries_evicted", before - st.live)

        s._evict_to = _evict_to
        s._lookahead_evict = _lookahead_evict
    return fp
