"""Per-layer orchestration of the read path (the reference session's fast path,
runtime/session.py:43-75, 430-467, 862-868, 1286-1460).

A session hands every sparse layer's attention to ``FastLayerPath``:

  * step 0 of a block (``step0``, session.py:1403-1454): split-K attention over
    [live prefix | block] keeping the prefix statistics, the prefix mass and the
    value-aware score of the selection rows, the read-set top-k with ascending indices
    and the gather of the selected entries into the layer's compact bf16 buffer;
  * every later denoising sub-step (``compact_attention``, session.py:1286-1336):
    attention over [selected entries | block];
  * look-ahead probes and prefill chunks (``attend``, session.py:1373-1401): block-causal
    split-K attention with the prefix mass of chosen rows.

Everything runs on the gfx950 kernels of libmaskahead_hip.so.  The sub-step attends
[compact | block] with split-K directly from the compact buffer and the block's own
K/V tensors: the reference first copies the block into the compact buffer and calls
SDPA over it; the result is the same softmax over the same entries.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .. import _native as N
from .._native import KernelUnavailableError
from ..kernels.splitk import Prefix, prefix_scores, splitk_attention
from ..kernels.step0 import Step0Buffers, step0_select


def fast_path_supported(config, head_dim: int, device_type: str = "cuda"):
    """(ok, reason): can this library's kernels serve `config` (session.py:43-75)?

    `config` is the reference's ExperimentConfig (or any object with the same
    attributes: backend, semantic, async_selector, collect_diagnostics,
    coverage_diagnostics, compact_format, attn_log_dir, selector, eviction, quant).
    Beyond the reference's own conditions, the bit widths and group sizes are those
    this library builds: 4-bit K and V with groups of 32, or 16-bit K and V."""
    import os

    cfg, sel, ev, q = config, config.selector, config.eviction, config.quant
    if os.environ.get("BITSIEVE_FAST", "1") == "0" or device_type != "cuda":
        return False, "disabled or not cuda"
    if cfg.backend == "torch" or cfg.semantic not in ("A", "dense"):
        return False, "backend/semantic"
    if cfg.async_selector and cfg.semantic == "A" and not ev.enabled and not sel.value_aware:
        return False, "async selector"
    if cfg.collect_diagnostics or cfg.coverage_diagnostics or cfg.compact_format != "bf16":
        return False, "diagnostics/compact format"
    if cfg.attn_log_dir:
        return False, "attention recording"
    if sel.score != "softmax" or sel.domain != "prefix" or sel.mode not in ("all", "middle"):
        return False, "selector score/domain/mode"
    if sel.value_joint or sel.value_per_query or sel.value_set != "none" or sel.value_caote:
        return False, "research selector"
    if sel.value_aware and sel.value_center != "attn":
        return False, "value centre"
    if ev.enabled and (ev.policy in ("greedy_set", "oracle_future", "ema_recent_score")
                       or ev.diag_path or ev.oracle_record_dir):
        return False, "research eviction"
    if not ((q.k_bits == 4 and q.v_bits == 4) or (q.k_bits == 16 and q.v_bits == 16)):
        return False, "bits"
    if q.k_bits == 4 and (q.key_token_group != 32 or q.value_channel_group != 32):
        return False, "group sizes"
    if getattr(q, "key_mode", "channel") != "channel" or getattr(q, "key_bias", "none") != "none" \
            or getattr(q, "rotation", "none") != "none":
        return False, "key transform"
    return head_dim in (64, 128), "head_dim"


def effective_topk(old_cache_len: int, topk: int, topk_percent: float | None = None, topk_floor: int | None = None):
    """Read budget of a block (config.py:172-183)."""
    import math

    if old_cache_len <= 0:
        return 0
    if topk_percent is not None:
        return min(old_cache_len, max(topk_floor or 1, int(math.ceil(old_cache_len * topk_percent / 100.0))))
    return min(old_cache_len, topk)


@dataclass
class CompactLayerState:
    """One layer's compact buffer (session.py:430-454): [B, Hkv, k + block, D]."""
    key: torch.Tensor
    value: torch.Tensor
    indices: torch.Tensor | None = None
    selected_k: int = 0


@dataclass
class FastLayerPath:
    """The fast path of one session over its PackedKVCache.

    cache: the session's PackedKVCache; block_size: tokens per block (the compact
    buffer's tail); query_indices: the block positions of the selection rows;
    value_aware / sort_indices: the selector's settings; slot_masks: optional uint8
    [B, Hkv, length] live masks per layer (0 = dead slot)."""

    cache: object
    block_size: int
    query_indices: list = field(default_factory=list)
    value_aware: bool = True
    sort_indices: bool = True
    compute_dtype: torch.dtype = torch.bfloat16
    dense_prefix_layers: int = 0
    semantic: str = "A"
    slot_masks: dict = field(default_factory=dict)
    states: dict = field(default_factory=dict)
    last_mass: dict = field(default_factory=dict)
    probe_mass: dict = field(default_factory=dict)
    chunk_mass: dict = field(default_factory=dict)
    qprobe_mass: dict = field(default_factory=dict)
    _rows_cache: tuple | None = None
    _prefix_cache: dict = field(default_factory=dict)
    _compact_prefix: dict = field(default_factory=dict)
    _planes_generation: int = -1
    _step0_bufs: dict = field(default_factory=dict)
    _step0_ws: Step0Buffers = field(default_factory=Step0Buffers)

    @property
    def head_dim(self) -> int:
        return self.cache.head_dim

    def prefix(self, layer_idx: int) -> Prefix:
        """session.py:1362-1367.  Kept per layer while the cache's planes (storage and
        strides), its lengths and the layer's slot mask are the ones it was built from: the
        descriptor holds nothing else, so a cache that grew, compacted, rebuilt or appended
        gives a new one (building the view and descriptor is most of a step's host time).
        When the cache has replaced its planes (planes_generation), every layer's kept
        descriptor is dropped at once, so none keeps the old planes alive."""
        c = self.cache
        gen = getattr(c, "planes_generation", 0)
        if gen != self._planes_generation:
            self._prefix_cache.clear()
            self._planes_generation = gen
        mask = self.slot_masks.get(layer_idx)
        key = (c.length, c.quantized_length, c.residual_length, id(mask),
               tuple((t.data_ptr(), t.stride()) if t is not None else None
                     for t in (c.k_q, c.k_scale, c.k_zero, c.v_q, c.v_scale, c.v_zero, c.k_residual, c.v_residual,
                               c.k_fp, c.v_fp)))
        hit = self._prefix_cache.get(layer_idx)
        if hit is not None and hit[0] == key and hit[2] is mask:
            return hit[1]
        pre = Prefix.from_view(c.layer_view(layer_idx))
        pre.mask = mask
        self._prefix_cache[layer_idx] = (key, pre, mask)
        return pre

    def rows(self, positions):
        """The selection rows to hand prefix_scores (session.py:1369-1376): positions 0 .. n-1
        in order stay a host list (the score kernels need no row table for them); any other
        list becomes an int32 device tensor, cached per distinct list."""
        key = tuple(int(p) for p in positions)
        if key == tuple(range(len(key))):
            return list(key)
        if self._rows_cache is None or self._rows_cache[0] != key:
            t = torch.tensor(key, dtype=torch.int32, device=self.cache.device)   # synchronous, kept
            self._rows_cache = (key, t)
        return self._rows_cache[1]

    def current_only(self, query, current_key, current_value, causal: int = 0, q_pos0: int = 0):
        """Attention over the block alone (session.py:1394-1401)."""
        out, _ = splitk_attention(query, Prefix(), current_key, current_value, scaling=self.head_dim ** -0.5,
                                  causal_block=causal, q_pos0=q_pos0, c_pos0=q_pos0)
        return out

    def attend(self, layer_idx, query, current_key, current_value, *, causal: int = 0, q_pos0: int = 0,
               mass_rows=None):
        """Attention over [live prefix | current], optionally with the prefix mass of
        mass_rows (session.py:1378-1392): look-ahead probes and prefill chunks."""
        prefix = self.prefix(layer_idx)
        if prefix.n == 0:
            return self.current_only(query, current_key, current_value, causal, q_pos0), None
        out, stats = splitk_attention(query, prefix, current_key, current_value, scaling=self.head_dim ** -0.5,
                                      causal_block=causal, q_pos0=q_pos0, c_pos0=q_pos0,
                                      want_prefix=mass_rows is not None)
        if mass_rows is None:
            return out, None
        rows = mass_rows if isinstance(mass_rows, torch.Tensor) else self.rows(mass_rows)
        mass, _ = prefix_scores(query, prefix, stats, rows, value=False, scaling=self.head_dim ** -0.5)
        return out, mass

    def probe(self, layer_idx, query, current_key, current_value, *, live_slots=None):
        """A lookahead probe forward on the fast path (session.py:2317-2332): the masked
        blocks k+1 .. k+M in one forward, block-causal over [live prefix | blocks] (block j
        reads blocks <= j).  The prefix mass of the queries of blocks k+2 .. (block
        positions block_size .. t-1) times the number of those blocks goes to
        probe_mass[layer_idx], in live order when live_slots [B, Hkv, live] (the eviction
        state's slots) is given (session.py:257-261)."""
        b = self.block_size
        t = query.shape[2]
        rows = list(range(b, t))
        out, mass = self.attend(layer_idx, query, current_key, current_value, causal=b, q_pos0=0,
                                mass_rows=rows if rows else None)
        if mass is not None:
            if live_slots is not None:
                mass = mass.gather(-1, live_slots.to(torch.int64))
            self.probe_mass[layer_idx] = mass * max(1, (t - b) // b)
        return out

    def prefill_chunk(self, layer_idx, query, current_key, current_value, *, want_mass: bool = False,
                      live_slots=None):
        """A prefill chunk on the fast path (session.py:1827-1876): block-causal attention
        over [live prefix | chunk]; with want_mass the prefix mass of every chunk position
        goes to chunk_mass[layer_idx] (live order when live_slots is given), the input of
        the EMA and chunk-wise lookahead policies."""
        t = query.shape[2]
        out, mass = self.attend(layer_idx, query, current_key, current_value, causal=self.block_size, q_pos0=0,
                                mass_rows=list(range(t)) if want_mass else None)
        if mass is not None:
            if live_slots is not None:
                mass = mass.gather(-1, live_slots.to(torch.int64))
            self.chunk_mass[layer_idx] = mass
        return out

    def ensure_state(self, layer_idx: int, selected_k: int) -> CompactLayerState:
        """session.py:438-454."""
        state = self.states.get(layer_idx)
        capacity = max(1, selected_k) + self.block_size
        if state is not None and state.key.shape[2] >= capacity:
            return state
        shape = (self.cache.batch_size, self.cache.num_kv_heads, capacity, self.head_dim)
        state = CompactLayerState(key=torch.empty(shape, device=self.cache.device, dtype=self.compute_dtype),
                                  value=torch.empty(shape, device=self.cache.device, dtype=self.compute_dtype))
        self.states[layer_idx] = state
        return state

    def step0(self, layer_idx, query, current_key, current_value, *, select: bool, topk: int,
              want_mass: bool = False, live_slots=None):
        """Step 0 of a block (session.py:1403-1454): attention over the live prefix and,
        when `select`, the block's read set of `topk` entries per KV head ranked by mass
        (or mass * ||v - c|| when value_aware), gathered into the compact buffer.  The
        prefix mass is kept in last_mass[layer_idx] when want_mass (eviction input): per
        physical slot, or in live order when live_slots [B, Hkv, live] (the eviction state's
        slots of this layer) is given, as the reference's _to_live (session.py:257-261)."""
        need_sel = select and bool(self.query_indices)
        need_mass = want_mass and bool(self.query_indices)
        prefix = self.prefix(layer_idx)
        if prefix.n == 0:
            return self.current_only(query, current_key, current_value, 0, 0)
        scale = self.head_dim ** -0.5
        if need_sel:
            # the whole step in one library call, into this layer's reused buffers (valid
            # until the layer's next step 0)
            k = min(int(topk), prefix.n)
            if k <= 0:
                raise ValueError("the read budget must be positive")
            if not self.sort_indices:
                raise KernelUnavailableError("the HIP read-set select returns ascending indices only "
                                             "(selector.sort_indices = False is not built)")
            state = self.ensure_state(layer_idx, k)
            bufs = self._step0_bufs.setdefault(layer_idx, Step0Buffers())
            out, _, mass, _, idx = step0_select(bufs, query, prefix, current_key, current_value,
                                                self.rows(self.query_indices), k, value=self.value_aware,
                                                scaling=scale, out_key=state.key[:, :, :k, :],
                                                out_value=state.value[:, :, :k, :], workspace=self._step0_ws)
            if need_mass:
                self.last_mass[layer_idx] = mass if live_slots is None else mass.gather(-1, live_slots.to(torch.int64))
            state.indices = idx
            state.selected_k = k
            return out
        out, stats = splitk_attention(query, prefix, current_key, current_value, scaling=scale,
                                      want_prefix=need_mass)
        if not need_mass:
            return out
        # a dense layer that keeps its prefix mass (eviction input)
        mass, _ = prefix_scores(query, prefix, stats, self.rows(self.query_indices), value=False, scaling=scale)
        self.last_mass[layer_idx] = mass if live_slots is None else mass.gather(-1, live_slots.to(torch.int64))
        return out

    def compact_attention(self, layer_idx, query, current_key, current_value):
        """A denoising sub-step: softmax attention over [selected entries | block]
        (session.py:1286-1336; sdpa_compact, reference.py:403-426)."""
        state = self.states.get(layer_idx)
        if state is None or state.selected_k <= 0:
            raise RuntimeError(f"layer {layer_idx} has no selected cache; finish_step0 was not called or "
                               "selection failed")
        k = state.selected_k
        ncur = current_key.shape[2]
        if k + ncur > state.key.shape[2]:
            raise RuntimeError("compact cache buffer capacity exceeded")
        cd = self.compute_dtype
        q, kc, vc = query.to(cd), current_key.to(cd), current_value.to(cd)
        stream = N.stream_of(q)
        key = (k, state.key.data_ptr(), state.value.data_ptr(), state.key.stride(), state.value.stride(),
               q.shape, q.stride(), kc.shape, kc.stride(), vc.stride(), stream)
        hit = self._compact_prefix.get(layer_idx)
        if hit is not None and hit[0] == key:
            # the same compact buffer, shapes and stream: the call checked and packed before,
            # with this call's operands and a fresh output
            args = hit[2]
            out = torch.empty_like(q)
            # the same shapes, strides and dtypes: only the operands' addresses change
            args[0].ptr, args[14].ptr = q.data_ptr(), out.data_ptr()
            if ncur:
                args[7].ptr, args[8].ptr = kc.data_ptr(), vc.data_ptr()
            N.check(N.load().ma_splitk_attention(*args), "ma_splitk_attention")
            return out.to(query.dtype)
        pre = Prefix.dense(state.key[:, :, :k, :], state.value[:, :, :k, :])
        out, _ = splitk_attention(q, pre, kc, vc, scaling=self.head_dim ** -0.5)
        # the arguments of that call, for the next sub-steps of this layer (splitk_attention's
        # own; the workspace is kept with them)
        b, hq, t, d = q.shape
        hkv, tc = kc.shape[1], kc.shape[2]
        ws_bytes = N.size_query("ma_splitk_workspace_bytes", b, hkv, hq, t, d, pre.nq, pre.nf, 0)
        ws = torch.empty((ws_bytes,), device=q.device, dtype=torch.uint8)
        args = [N.t4(q), b, hq, t, d, pre.native(), hkv, N.t4(kc if tc else None), N.t4(vc if tc else None), tc, 0, 0,
                0, float(self.head_dim ** -0.5), N.t4(out), None, None, None, 0, ws.data_ptr(), ws_bytes, stream]
        self._compact_prefix[layer_idx] = (key, pre, args, ws)
        return out.to(query.dtype)

    def question_probe(self, layer_idx, query, current_key, current_value, *, q_pos0: int, live_slots=None):
        """A question-probe forward (session.py:2289-2297): block-causal attention from block
        position q_pos0 over [live prefix | probe tokens]; the prefix mass of every probe
        query goes to qprobe_mass[layer_idx] (live order when live_slots is given)."""
        t = query.shape[2]
        out, mass = self.attend(layer_idx, query, current_key, current_value, causal=self.block_size,
                                q_pos0=q_pos0, mass_rows=list(range(t)))
        if mass is not None:
            self.qprobe_mass[layer_idx] = mass if live_slots is None else mass.gather(-1, live_slots.to(torch.int64))
        return out

    def dense_required(self, layer_idx: int, ctx: "BlockContext") -> bool:
        """Whether this layer attends the whole live prefix instead of a read set
        (session.py:456-467)."""
        if self.semantic == "dense" or layer_idx < self.dense_prefix_layers:
            return True
        if ctx.evicting:
            return ctx.live_len == 0 or not self.query_indices
        return ctx.old_cache_len == 0 or ctx.topk >= ctx.old_cache_len or not self.query_indices

    def route(self, layer_idx, query, current_key, current_value, ctx: "BlockContext"):
        """One layer's attention call on the fast path, sent where the reference session's
        attend hook sends it (_attend_entry / _attend_main, session.py:2281-2418): a prefill
        chunk, a question probe, a lookahead probe, step 0 of a block (dense layers: the
        attention, and the mass when wanted; sparse layers: also the read set), or a later
        denoising sub-step (dense layers: over the live prefix; sparse layers: over the
        read set)."""
        live = None if ctx.live_slots is None else ctx.live_slots.get(layer_idx)
        if ctx.prefill:
            return self.prefill_chunk(layer_idx, query, current_key, current_value, want_mass=ctx.want_mass,
                                      live_slots=live)
        if ctx.qprobe_start is not None:
            return self.question_probe(layer_idx, query, current_key, current_value, q_pos0=ctx.qprobe_start,
                                       live_slots=live)
        if ctx.probe:
            return self.probe(layer_idx, query, current_key, current_value, live_slots=live)
        dense = self.dense_required(layer_idx, ctx)
        if ctx.step_index == 0:
            return self.step0(layer_idx, query, current_key, current_value,
                              select=not dense and self.semantic == "A", topk=ctx.topk, want_mass=ctx.want_mass,
                              live_slots=live)
        if dense:
            return self.attend(layer_idx, query, current_key, current_value)[0]
        return self.compact_attention(layer_idx, query, current_key, current_value)


@dataclass
class BlockContext:
    """The session state one layer call is routed on (the reference session's fields).

    step_index: denoising step within the block (0 = the step that selects);
    probe: a lookahead probe forward (session._probe); prefill: a prefill-chunk forward
    (session._prefill_mode); qprobe_start: block position of a question probe, or None;
    old_cache_len: prefix length when the block began; topk: the block's read budget
    (config.effective_topk); evicting: eviction is on, so the cache is the live set;
    live_len: live entries per lane; want_mass: step 0 / the chunk keeps its prefix mass
    (lookahead pending, EMA policies); live_slots: per layer, the eviction state's slots
    [B, Hkv, live] that put masses in live order (None: per physical slot)."""

    step_index: int = 0
    probe: bool = False
    prefill: bool = False
    qprobe_start: int | None = None
    old_cache_len: int = 0
    topk: int = 0
    evicting: bool = False
    live_len: int = 0
    want_mass: bool = False
    live_slots: dict | None = None
