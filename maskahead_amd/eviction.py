"""Bounded KV cache: the eviction configuration and the per-lane live-entry state.

Drop-in for the reference's ``maskahead.eviction`` on the paths the GPU keep step uses
(eviction.py:55-457).  ``EvictionConfig`` keeps the reference's field names, defaults and
validation so the same YAML files load; ``EvictionState`` keeps its arrays (g, n, pos,
phys per (layer, batch, KV head) lane, live axis last) on the GPU, and its two hot
operations run in gfx950 kernels:

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
    """Per (layer, batch, KV head) live-entry state (eviction.py:205-457): g f32, n int16,
    pos int32 (int64 when max_position >= 2^31), phys int32, shape [L, B, Hkv, capacity],
    the first ``live`` slots in use and ordered by position."""

    def __init__(self, *, num_layers: int, batch_size: int, num_kv_heads: int, capacity: int,
                 device: torch.device | str, max_position: int = 1 << 31) -> None:
        self.num_layers = int(num_layers)
        self.batch_size = int(batch_size)
        self.num_kv_heads = int(num_kv_heads)
        self.device = torch.device(device)
        self.pos_dtype = torch.int32 if max_position < (1 << 31) else torch.int64
        shape = (self.num_layers, self.batch_size, self.num_kv_heads, capacity)
        self.g = torch.zeros(shape, dtype=torch.float32, device=self.device)
        self.n = torch.zeros(shape, dtype=torch.int16, device=self.device)
        self.pos = torch.zeros(shape, dtype=self.pos_dtype, device=self.device)
        self.phys = torch.zeros(shape, dtype=torch.int32, device=self.device)
        self.live = 0
        self._capacity = capacity
        self.pin: tuple[int | torch.Tensor, int] | None = None

    # -- growth ------------------------------------------------------------
    def _grow_to(self, needed: int) -> None:
        if needed <= self._capacity:
            return
        new_cap = max(needed, self._capacity * 2, 1)
        pad = new_cap - self._capacity
        shape = (self.num_layers, self.batch_size, self.num_kv_heads, pad)

        def grow(t):
            return torch.cat([t, torch.zeros(shape, dtype=t.dtype, device=self.device)], -1)

        self.g, self.n, self.pos, self.phys = grow(self.g), grow(self.n), grow(self.pos), grow(self.phys)
        self._capacity = new_cap

    def append(self, positions, phys: torch.Tensor | None = None) -> None:
        """Admit new entries with g = 0, n = 0 (eviction.py:258-281)."""
        if isinstance(positions, range):
            positions = list(positions)
        if isinstance(positions, list):
            positions = torch.tensor(positions, dtype=self.pos_dtype, device=self.device)
        m = int(positions.numel())
        if m == 0:
            return
        self._grow_to(self.live + m)
        sl = slice(self.live, self.live + m)
        self.g[..., sl] = 0.0
        self.n[..., sl] = 0
        self.pos[..., sl] = positions.to(self.pos_dtype).view(1, 1, 1, m)
        self.phys[..., sl] = (positions if phys is None else phys).to(self.phys.dtype).view(1, 1, 1, m)
        self.live += m

    # -- update ------------------------------------------------------------
    def observe(self, layer_idx: int, alpha: torch.Tensor, decay: float, weight: float = 1.0) -> None:
        """Fold a block's attention mass into the EMA of one layer (eviction.py:284-308)."""
        if self.live == 0:
            return
        if alpha.shape[-1] != self.live:
            raise ValueError(f"alpha has {alpha.shape[-1]} entries but {self.live} are live; "
                             "the selector must rank exactly the live set")
        sl = slice(0, self.live)
        g = self.g[layer_idx, ..., sl]
        if decay == 1.0:
            g.add_(alpha.to(g.dtype), alpha=float(weight))
        else:
            g.mul_(decay).add_(alpha.to(g.dtype), alpha=1.0 - decay)
        self.n[layer_idx, ..., sl] += 1

    def corrected(self, layer_idx: int, decay: float) -> torch.Tensor:
        """ghat = g / (1 - decay**n), 0 where n == 0 (eviction.py:310-322)."""
        sl = slice(0, self.live)
        g = self.g[layer_idx, ..., sl]
        n = self.n[layer_idx, ..., sl]
        if decay in (0.0, 1.0):
            return g.clone()
        denom = 1.0 - torch.pow(torch.tensor(decay, dtype=torch.float32, device=g.device), n.to(torch.float32))
        return torch.where(n > 0, g / denom.clamp_min(1e-8), torch.zeros_like(g))

    # -- eviction ----------------------------------------------------------
    def survivors(self, cfg: EvictionConfig, capacity: int, value_spread: torch.Tensor | None = None,
                  score: torch.Tensor | None = None) -> torch.Tensor:
        """Live-axis indices to keep, [L, B, Hkv, capacity], in position order
        (eviction.py:325-409).  Every policy reduces to one ma_keep_select launch over
        all lanes: a recency window that is always kept, plus the top of a rank among
        the rest where sinks and pinned positions rank +inf."""
        sl = slice(0, self.live)
        pos = self.pos[..., sl]
        if cfg.policy == "recent":
            # the C newest, sinks and pins first: rank by position, window 0
            rank = pos.to(torch.float32)
            return keep_select(pos, rank, capacity, 0, sink_tokens=cfg.sink_tokens, pin=self._pin_rows())
        if cfg.policy == "snapkv":
            if score is None or score.shape != self.g.shape[:3] + (self.live,):
                raise ValueError("policy snapkv needs a [L, B, Hkv, live] score")
            return keep_select(pos, score.to(torch.float32), capacity, cfg.snapkv_window,
                               sink_tokens=cfg.sink_tokens, pin=self._pin_rows())
        if cfg.policy in ("ema_recent", "ema_recent_value", "ema_recent_score") + _SCORED:
            w = min(cfg.recent_window, capacity)
            if capacity - w > 0:
                ghat = torch.stack([self.corrected(l, cfg.decay) for l in range(self.num_layers)], dim=0)
                if cfg.policy in _SCORED:
                    if score is None or score.shape != ghat.shape:
                        raise ValueError(f"policy {cfg.policy} needs a [L, B, Hkv, live] score")
                    ghat = score.to(ghat.dtype)
                if cfg.policy == "ema_recent_value":
                    if value_spread is None:
                        raise ValueError("policy ema_recent_value needs value_spread; the caller must supply "
                                         "per-entry ||v - vbar||")
                    if value_spread.shape != ghat.shape:
                        raise ValueError(f"value_spread has shape {tuple(value_spread.shape)} but the live EMA "
                                         f"is {tuple(ghat.shape)}")
                    if cfg.value_caote:
                        norm = ghat / ghat.sum(dim=-1, keepdim=True).clamp_min(1e-12)
                        ghat = norm / (1.0 - norm).clamp_min(1e-6)
                    ghat = ghat * value_spread.to(ghat.dtype)
            else:
                ghat = torch.zeros(pos.shape, dtype=torch.float32, device=self.device)
            return keep_select(pos, ghat.contiguous(), capacity, w, sink_tokens=cfg.sink_tokens,
                               pin=self._pin_rows())
        raise ValueError(f"policy {cfg.policy} does not evict")

    def _pin_rows(self):
        if self.pin is None:
            return None
        lo, hi = self.pin
        if isinstance(lo, torch.Tensor):
            lo = lo.to(self.device, torch.int64).view(1, -1, 1)
        return (lo, hi)

    def compact(self, keep: torch.Tensor) -> None:
        """Drop everything outside ``keep`` [L, B, Hkv, C], in place (eviction.py:411-418)."""
        c = keep.shape[-1]
        lb = self.num_layers * self.batch_size
        h = self.num_kv_heads
        k3 = keep.reshape(lb, h, c)
        planes = [t.view(lb, h, t.shape[-1], 1) for t in (self.g, self.n, self.pos, self.phys)]
        compact_tokens(planes, k3, self.live)
        self.live = c

    def maybe_evict(self, cfg: EvictionConfig, *, block_index: int, tokens_seen: int,
                    value_spread_fn: Callable[[], torch.Tensor] | None = None,
                    score_fn: Callable[[], torch.Tensor] | None = None) -> torch.Tensor | None:
        """Evict on schedule (eviction.py:420-457); returns the survivors or None."""
        if not cfg.enabled or self.live == 0 or cfg.policy == "snapkv":
            return None
        if (block_index + 1) % cfg.interval_blocks:
            return None
        capacity = cfg.capacity(tokens_seen)
        if self.live <= capacity:
            return None
        spread = None
        if cfg.policy == "ema_recent_value":
            if value_spread_fn is None:
                raise ValueError("policy ema_recent_value needs a value_spread_fn")
            spread = value_spread_fn()
        score = None
        if cfg.policy in ("expected_attention", "greedy_set", "oracle_future", "snapkv"):
            if score_fn is None:
                raise ValueError(f"policy {cfg.policy} needs a score_fn")
            score = score_fn(capacity) if cfg.policy == "greedy_set" else score_fn()
        keep = self.survivors(cfg, capacity, spread, score)
        self.compact(keep)
        return keep
