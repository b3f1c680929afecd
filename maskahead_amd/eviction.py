"""Bounded KV cache: the eviction configuration and the per-lane live-entry state.

Drop-in for the reference's ``maskahead.eviction`` on the paths the GPU keep step uses
(eviction.py:55-457).  ``EvictionConfig`` keeps the reference's field names, defaults and
validation so the same YAML files load (an interface); ``EvictionState`` is a column
store of the live entries of every (layer, batch, KV head) lane on the GPU, and its two
hot operations run in gfx950 kernels:

    keep = state.survivors(cfg, capacity, spread, score)   # ma_keep_select
    state.compact(keep)                                    # ma_compact_tokens, in place

The EMA bookkeeping (observe / corrected) is element-wise arithmetic on those arrays
and stays in torch ops on the same device.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Literal

import torch

from .kernels.keep import compact_tokens, keep_select

Policy = Literal["none", "recent", "ema_recent", "ema_recent_value", "ema_recent_score", "expected_attention",
                 "greedy_set", "oracle_future", "lookahead", "snapkv"]

_POLICIES = ("none", "recent", "ema_recent", "ema_recent_value", "ema_recent_score", "expected_attention",
             "greedy_set", "oracle_future", "lookahead", "snapkv")
_SCORED = ("expected_attention", "greedy_set", "oracle_future", "lookahead")
_EMA_POLICIES = ("ema_recent", "ema_recent_value", "ema_recent_score")


@dataclass(slots=True)
class EvictionConfig:
    """Eviction settings (eviction.py:55-202): same fields, defaults and checks, so the
    reference's configuration files load unchanged."""

    policy: Policy = "none"
    decay: float = 0.9
    recent_window: int = 128
    capacity_percent: float = 5.0
    capacity_floor: int = 256
    interval_blocks: int = 4
    value_center: Literal["mean", "attn", "none"] = "mean"
    value_caote: bool = False
    ea_horizon: int = 128
    ea_decay: float = 0.9
    ea_eps: float = 0.02
    ea_diag: bool = False
    diag_path: str | None = None
    greedy_chunk: int = 8
    oracle_record_dir: str | None = None
    oracle_dir: str | None = None
    oracle_horizon: int = 4
    record_only: bool = False
    snapkv_window: int = 32
    snapkv_pool_kernel: int = 5
    sink_tokens: int = 0
    lookahead_blocks: int = 1
    lookahead_probe: str = "mask"
    lookahead_score: str = "value"
    lookahead_merge: bool = False
    prefill_chunk: int = 0
    prefill_capacity_percent: float | None = None
    prefill_question_probe: bool = False
    pin_question: bool = False
    compaction: str = "lazy"
    repack_below: float = 1.0
    stage_bf16: str = "none"

    @property
    def enabled(self) -> bool:
        return self.policy != "none"

    @property
    def horizon_blocks(self) -> int:
        return self.lookahead_blocks if self.lookahead_blocks > 0 else self.interval_blocks

    def capacity(self, tokens_seen: int) -> int:
        """C = max(capacity_percent % of every token the cache has held, capacity_floor)
        (eviction.py:200-202)."""
        return max(int(self.capacity_percent / 100.0 * tokens_seen), self.capacity_floor)

    def validate(self) -> None:
        """The reference's checks (eviction.py:165-194), same messages."""
        if self.policy not in _POLICIES:
            raise ValueError(f"unknown eviction policy: {self.policy}")
        if self.prefill_question_probe and self.policy != "lookahead":
            raise ValueError("prefill_question_probe ranks with the lookahead score; use policy lookahead")
        if not 0.0 <= self.decay <= 1.0:
            raise ValueError(f"decay must be in [0, 1] (1 = H2O accumulated sum), got {self.decay}")
        if self.recent_window < 0:
            raise ValueError("recent_window must be non-negative")
        if self.capacity_floor <= 0:
            raise ValueError("capacity_floor must be positive")
        if not 0.0 < self.capacity_percent <= 100.0:
            raise ValueError("capacity_percent must be in (0, 100]")
        if self.interval_blocks <= 0:
            raise ValueError("interval_blocks must be positive")
        if self.snapkv_window <= 0 or self.snapkv_pool_kernel <= 0 or self.snapkv_pool_kernel % 2 == 0:
            raise ValueError("SnapKV window must be positive and pooling kernel must be positive and odd")
        if self.value_center not in ("mean", "attn", "none"):
            raise ValueError(f"unknown eviction value_center: {self.value_center}")
        if self.ea_horizon <= 0 or not 0.0 <= self.ea_decay < 1.0 or self.ea_eps < 0.0:
            raise ValueError("bad expected_attention parameters")
        if (self.policy.startswith("ema_recent") or self.policy in _SCORED) and \
                self.recent_window > self.capacity_floor:
            raise ValueError(
                f"recent_window={self.recent_window} exceeds capacity_floor={self.capacity_floor}; the window "
                "alone would fill the budget and no entry could ever be kept on its EMA")


class EvictionState:
    """The live set of every (layer, batch, KV head) lane, as columns on the GPU.

    Four columns, each [L, B, Hkv, rows] with the live axis last and the first ``live``
    rows in use, ordered by position (the reference's EvictionState arrays,
    eviction.py:205-281): ``g`` f32 attention EMA, ``n`` int16 observation count, ``pos``
    token position (int32, int64 when max_position >= 2^31), ``phys`` the entry's physical
    slot in the cache.  Every lane of a state holds the same number of live entries.

    Keep-set selection reduces every policy to one contest -- a recency window kept
    outright plus the top of a per-entry rank among the rest, sinks and pinned positions
    ranking +inf -- solved for all lanes in one ma_keep_select call; compaction moves the
    four columns in one ma_compact_tokens call."""

    _COLUMNS = ("g", "n", "pos", "phys")

    def __init__(self, *, num_layers: int, batch_size: int, num_kv_heads: int, capacity: int,
                 device: torch.device | str, max_position: int = 1 << 31) -> None:
        self.num_layers, self.batch_size, self.num_kv_heads = int(num_layers), int(batch_size), int(num_kv_heads)
        self.device = torch.device(device)
        self.pos_dtype = torch.int32 if max_position < (1 << 31) else torch.int64
        self._dtypes = {"g": torch.float32, "n": torch.int16, "pos": self.pos_dtype, "phys": torch.int32}
        self._cols: dict[str, torch.Tensor] = {}
        self.live = 0
        self.pin: tuple[int | torch.Tensor, int] | None = None
        # sink statistic of the evictions (eviction.py:446-451): lanes that dropped one of
        # positions 0..3, counted on the device (read back only when asked for), and lanes
        # evicted in all
        self._sink_drops: torch.Tensor | None = None
        self.lanes_evictions = 0
        self._ensure(max(int(capacity), 1))

    # the columns, as attributes (views of the whole storage; rows >= live are unused)
    g = property(lambda self: self._cols["g"])
    n = property(lambda self: self._cols["n"])
    pos = property(lambda self: self._cols["pos"])
    phys = property(lambda self: self._cols["phys"])

    @property
    def sink_lanes_evicted(self) -> int:
        """(layer, batch, KV head) lane evictions so far that dropped a position < 4."""
        return 0 if self._sink_drops is None else int(self._sink_drops.item())

    def state_nbytes(self) -> int:
        """Bytes of the policy's own per-entry state -- the EMA, its observation count and
        the position of every live entry of every lane (eviction.py:460-466)."""
        per_entry = sum(self._cols[name].element_size() for name in ("g", "n", "pos"))
        return self.num_layers * self.batch_size * self.num_kv_heads * self.live * per_entry

    @property
    def rows(self) -> int:
        return int(self._cols["pos"].shape[-1])

    def _ensure(self, rows: int) -> None:
        """At least `rows` rows per lane (doubling), live rows kept, new rows zero."""
        have = self.rows if self._cols else 0
        if rows <= have:
            return
        rows = max(rows, 2 * have)
        lead = (self.num_layers, self.batch_size, self.num_kv_heads)
        for name in self._COLUMNS:
            col = torch.zeros(lead + (rows,), dtype=self._dtypes[name], device=self.device)
            if self.live:
                col[..., :self.live] = self._cols[name][..., :self.live]
            self._cols[name] = col

    def _in_use(self, name: str, layer: int | None = None) -> torch.Tensor:
        col = self._cols[name]
        return col[..., :self.live] if layer is None else col[layer, ..., :self.live]

    # -- admission and observation -------------------------------------------------------------
    def append(self, positions, phys: torch.Tensor | None = None) -> None:
        """Admit entries at `positions` (the same in every lane, increasing, after every
        live position): EMA 0, never observed, slot = `phys` or the position."""
        p = torch.as_tensor(list(positions) if isinstance(positions, range) else positions, device=self.device)
        m = int(p.numel())
        if m == 0:
            return
        self._ensure(self.live + m)
        rows = slice(self.live, self.live + m)
        fill = {"g": 0, "n": 0, "pos": p.view(1, 1, 1, m), "phys": (p if phys is None else phys).view(1, 1, 1, m)}
        for name, value in fill.items():
            self._cols[name][..., rows] = value
        self.live += m

    def observe(self, layer_idx: int, alpha: torch.Tensor, decay: float, weight: float = 1.0) -> None:
        """Fold one block's attention mass alpha [B, Hkv, live] of layer `layer_idx` into its
        EMA: g <- decay * g + (1 - decay) * alpha, or g <- g + weight * alpha when decay is
        1 (H2O's accumulated attention over `weight` queries); n counts the observations.
        The torch operations are the reference's (eviction.py:284-308, scale then add the
        weighted mass), so that g has the same bits."""
        if self.live == 0:
            return
        if alpha.shape[-1] != self.live:
            raise ValueError(f"alpha has {alpha.shape[-1]} entries but {self.live} are live; "
                             "the selector must rank exactly the live set")
        g = self._in_use("g", layer_idx)
        a = alpha.to(torch.float32)
        if decay == 1.0:
            g.add_(a, alpha=float(weight))
        else:
            g.mul_(decay).add_(a, alpha=1.0 - decay)
        self._in_use("n", layer_idx).add_(1)

    def corrected(self, layer_idx: int, decay: float) -> torch.Tensor:
        """The bias-corrected EMA g / (1 - decay^n) of one layer, 0 where never observed
        (eviction.py:310-322); g itself when decay is 0 or 1."""
        g, n = self._in_use("g", layer_idx), self._in_use("n", layer_idx)
        if decay in (0.0, 1.0):
            return g.clone()
        seen = n > 0
        scale = 1.0 - torch.pow(torch.tensor(decay, dtype=torch.float32, device=g.device), n.to(torch.float32))
        return torch.where(seen, g / scale.clamp_min(1e-8), torch.zeros_like(g))

    # -- keep-set selection ----------------------------------------------------------------------
    def _contest(self, cfg: EvictionConfig, capacity: int, value_spread, score) -> tuple[torch.Tensor, int]:
        """(rank [L, B, Hkv, live] f32, window) of a policy (eviction.py:325-409): the window's
        newest entries are kept outright, the rest of the budget goes to the highest rank."""
        live_shape = (self.num_layers, self.batch_size, self.num_kv_heads, self.live)
        policy = cfg.policy
        if policy == "recent":                        # StreamingLLM: the newest (+ sinks, pins)
            return self._in_use("pos").to(torch.float32), 0
        if policy == "snapkv":                        # its observation window + pooled attention
            if score is None or tuple(score.shape) != live_shape:
                raise ValueError("policy snapkv needs a [L, B, Hkv, live] score")
            return score.to(torch.float32), cfg.snapkv_window
        if policy not in _EMA_POLICIES + _SCORED:
            raise ValueError(f"policy {policy} does not evict")
        window = min(cfg.recent_window, capacity)
        if capacity == window:                        # the window is the whole budget
            return torch.zeros(live_shape, dtype=torch.float32, device=self.device), window
        if policy in _SCORED:
            if score is None or tuple(score.shape) != live_shape:
                raise ValueError(f"policy {policy} needs a [L, B, Hkv, live] score")
            return score.to(torch.float32), window
        rank = torch.stack([self.corrected(layer, cfg.decay) for layer in range(self.num_layers)])
        if policy == "ema_recent_value":
            if value_spread is None:
                raise ValueError("policy ema_recent_value needs value_spread; the caller must supply "
                                 "per-entry ||v - vbar||")
            if tuple(value_spread.shape) != live_shape:
                raise ValueError(f"value_spread has shape {tuple(value_spread.shape)} but the live EMA "
                                 f"is {live_shape}")
            if cfg.value_caote:
                share = rank / rank.sum(dim=-1, keepdim=True).clamp_min(1e-12)
                rank = share / (1.0 - share).clamp_min(1e-6)
            rank = rank * value_spread.to(rank.dtype)
        return rank, window

    def survivors(self, cfg: EvictionConfig, capacity: int, value_spread: torch.Tensor | None = None,
                  score: torch.Tensor | None = None, check: bool = True) -> torch.Tensor:
        """Live-axis indices of the `capacity` entries to keep in every lane, [L, B, Hkv, C],
        in position order: the policy's contest solved by ma_keep_select.  check=False skips
        the read-back of the positions' order check (append admits increasing positions
        after the live ones, so the state keeps them ascending)."""
        rank, window = self._contest(cfg, capacity, value_spread, score)
        return keep_select(self._in_use("pos"), rank.contiguous(), capacity, window, sink_tokens=cfg.sink_tokens,
                           pin=self._pin_rows(), check=check)

    def _pin_rows(self):
        """The pinned position range (lo, hi): lo an int or a per-sequence [B] tensor."""
        if self.pin is None:
            return None
        lo, hi = self.pin
        if isinstance(lo, torch.Tensor):
            lo = lo.to(self.device, torch.int64).view(1, -1, 1)
        return lo, hi

    def compact(self, keep: torch.Tensor) -> None:
        """Keep the live rows keep [L, B, Hkv, C] of every column, in that order, in place."""
        c = int(keep.shape[-1])
        lanes, h = self.num_layers * self.batch_size, self.num_kv_heads
        planes = [self._cols[name].view(lanes, h, self.rows, 1) for name in self._COLUMNS]
        compact_tokens(planes, keep.reshape(lanes, h, c), self.live)
        self.live = c

    def maybe_evict(self, cfg: EvictionConfig, *, block_index: int, tokens_seen: int,
                    value_spread_fn: Callable[[], torch.Tensor] | None = None,
                    score_fn: Callable[[], torch.Tensor] | None = None) -> torch.Tensor | None:
        """The end-of-block eviction of the EMA and scored policies (eviction.py:420-457):
        every interval_blocks blocks, when more than cfg.capacity(tokens_seen) entries are
        live, keep that many and compact; returns the keep set, or None when nothing ran.
        SnapKV compresses the prompt only and never evicts here."""
        due = cfg.enabled and cfg.policy != "snapkv" and (block_index + 1) % cfg.interval_blocks == 0
        capacity = cfg.capacity(tokens_seen)
        if not due or self.live <= capacity:
            return None
        spread = score = None
        if cfg.policy == "ema_recent_value":
            if value_spread_fn is None:
                raise ValueError("policy ema_recent_value needs a value_spread_fn")
            spread = value_spread_fn()
        if cfg.policy in ("expected_attention", "greedy_set", "oracle_future"):
            if score_fn is None:
                raise ValueError(f"policy {cfg.policy} needs a score_fn")
            score = score_fn(capacity) if cfg.policy == "greedy_set" else score_fn()
        keep = self.survivors(cfg, capacity, spread, score)
        self._count_sink_drops(keep)
        self.compact(keep)
        return keep

    def _count_sink_drops(self, keep: torch.Tensor) -> None:
        """Add the lanes whose keep set drops one of positions 0..3 (before compact)."""
        sinks = self._in_use("pos") < 4
        kept = torch.gather(sinks, -1, keep).sum(-1)
        drops = (kept < sinks.sum(-1)).sum()
        self._sink_drops = drops if self._sink_drops is None else self._sink_drops + drops
        self.lanes_evictions += int(sinks[..., 0].numel())


def live_cache_nbytes(pos: torch.Tensor, *, live: int, head_dim: int, k_bits: int, v_bits: int,
                      key_token_group: int, value_channel_group: int, param_bytes: int = 2,
                      compute_bytes: int = 2) -> int:
    """Bytes a cache holding exactly the live set pos[..., :live] would occupy
    (eviction.py:468-516): the packed or 16-bit payload of every live entry; for packed
    keys one scale/zero vector per key group that still holds a live entry (a group lives
    while any of its entries does), for packed values one per entry and value group.
    pos: [L, B, Hkv, rows] positions, the first `live` of each lane valid, any order."""
    if live <= 0:
        return 0
    lanes = pos.shape[0] * pos.shape[1] * pos.shape[2]
    entries = lanes * live
    if k_bits >= 16:
        k_bytes = entries * head_dim * compute_bytes
    else:
        grp = torch.sort(pos[..., :live].reshape(lanes, live) // key_token_group, dim=-1).values
        groups = lanes + int((grp[:, 1:] != grp[:, :-1]).sum())      # distinct groups per lane, summed
        k_bytes = entries * head_dim * k_bits // 8 + groups * head_dim * 2 * param_bytes
    if v_bits >= 16:
        v_bytes = entries * head_dim * compute_bytes
    else:
        v_bytes = entries * head_dim * v_bits // 8 + entries * (head_dim // value_channel_group) * 2 * param_bytes
    return k_bytes + v_bytes
