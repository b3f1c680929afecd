"""Per-layer KV store of the read/keep path, in the reference's storage format.

``PackedKVCache`` holds every layer's tokens in the layouts the kernels read -- the
format of the reference's ``maskahead.cache`` (cache.py:142-189), which is an interface
here: the same tensor names, shapes and capacity-padded strides, the same nibble order,
the same logical length (``dropped`` entries after a compaction) and the same append
protocol the model hooks drive (begin_append / stage_layer / commit_append,
cache.py:385-566).

How this store is organised is its own: every stored array is a *plane* with a unit --
one row per token, per 32-token key group, or per residual (bf16 tail) token -- and
growth, compaction bookkeeping and memory accounting are driven from that table.  The
data movement runs on the gfx950 kernels: the bf16 block append (ma_append_tokens), the
4-bit quantizers (ma_quantize_keys / ma_quantize_values), the dequant
(ma_dequant_prefix), the gather (ma_gather_kv), compaction in place (ma_compact_tokens)
and the packed lazy rebuild of every layer in one launch (ma_rebuild_packed).

Built for 4-bit K/V (key groups of 32 tokens per channel, value groups of 32 channels
per token, f16 scale / zero) and 16-bit K/V; other valid settings raise
KernelUnavailableError.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _native as N
from ._native import KernelUnavailableError
from .config import QuantizationConfig
from .kernels.keep import append_tokens, compact_tokens

_PARAM_DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}

# plane name -> unit of its axis 3: "tok" (one row per stored token of a 16-bit store),
# "qtok" (one row per quantized token), "grp" (one row per quantized key group), "res"
# (one row per bf16 residual token of a packed store)
_UNITS = {"k_fp": "tok", "v_fp": "tok", "v_q": "qtok", "v_scale": "qtok", "v_zero": "qtok",
          "k_q": "grp", "k_scale": "grp", "k_zero": "grp", "k_residual": "res", "v_residual": "res"}


@dataclass(slots=True)
class AppendPlan:
    """An append in progress (the reference's AppendPlan, cache.py:27-34): the length it
    starts from, the new tokens, the residual before, how many tail tokens become whole
    quantized key groups and the residual after, and which layers are written."""
    old_length: int
    new_tokens: int
    old_residual: int
    quantize_from_residual: int
    new_residual: int
    staged_layers: set[int]


@dataclass(slots=True)
class LayerCacheView:
    """One layer's stored prefix, as views (the reference's LayerCacheView, cache.py:37-60)."""
    k_bits: int
    v_bits: int
    length: int
    quantized_length: int
    residual_length: int
    key_token_group: int
    value_channel_group: int
    k_q: torch.Tensor | None
    k_scale: torch.Tensor | None
    k_zero: torch.Tensor | None
    v_q: torch.Tensor | None
    v_scale: torch.Tensor | None
    v_zero: torch.Tensor | None
    k_fp: torch.Tensor | None
    v_fp: torch.Tensor | None
    k_residual: torch.Tensor | None
    v_residual: torch.Tensor | None
    head_dim: int | None = None
    key_mode: str = "channel"
    k_chan: torch.Tensor | None = None


def _dynamic_layer(dyn, layer: int):
    """(K, V) of one layer of a prefill cache object, through the first access it offers
    (the transformers cache APIs: tuple indexing; key_cache / value_cache lists; 5.x
    layers[i].keys / .values); TypeError when none yields both tensors."""
    kv = None
    try:
        k, v = dyn[layer]
        kv = (k, v)
    except Exception:
        if hasattr(dyn, "key_cache"):
            kv = (dyn.key_cache[layer], dyn.value_cache[layer])
        elif hasattr(dyn, "layers"):
            kv = (dyn.layers[layer].keys, dyn.layers[layer].values)
    if kv is None or kv[0] is None or kv[1] is None:
        raise TypeError(f"cannot read layer {layer} out of {type(dyn).__name__}")
    return kv


def _ceil_to(x: int, m: int) -> int:
    return -(-x // m) * m


class PackedKVCache:
    """[L, B, Hkv, rows, ...] planes of every layer (see the module docstring).

    length = entries stored; of these the first quantized_length are 4-bit (whole key
    groups) and the last residual_length bf16 (packed caches), or all are 16-bit.
    get_seq_length() = length + dropped is the next position."""

    _START_TOKENS = 2048          # first token capacity (rows), before any growth
    _GROWTH = 1.5

    def __init__(self, *, num_layers: int, batch_size: int, num_kv_heads: int, head_dim: int, max_tokens: int,
                 quant: QuantizationConfig, device: torch.device | str, compute_dtype: torch.dtype = torch.bfloat16,
                 backend: str = "auto") -> None:
        quant.validate(head_dim=head_dim)
        if min(num_layers, batch_size, num_kv_heads, head_dim) <= 0:
            raise ValueError("all cache dimensions must be positive")
        if backend not in ("auto", "triton", "torch", "hip"):
            raise ValueError(f"unknown cache backend: {backend}")
        if backend == "torch":
            raise KernelUnavailableError("backend='torch' is the reference's CPU path; this cache runs on the "
                                         "HIP kernels only")
        quant.require_built()
        self.num_layers, self.batch_size = int(num_layers), int(batch_size)
        self.num_kv_heads, self.head_dim = int(num_kv_heads), int(head_dim)
        self.max_tokens = int(max_tokens)
        self.quant = quant
        self.device = torch.device(device)
        self.compute_dtype = compute_dtype
        self.param_dtype = _PARAM_DTYPES[quant.param_dtype]
        self.backend = backend
        self.length = self.quantized_length = self.residual_length = self.dropped = 0
        self.stage = False            # True: appended tokens stay bf16 until a rebuild quantizes them
        self.rotation = self.key_center = self.k_chan = None
        self.peak_used_bytes = self.peak_allocated_bytes = 0
        self.memory_trace: list[list[int]] | None = None
        self._append_plan: AppendPlan | None = None
        # bumped whenever the planes are replaced (growth, shrink after compaction): holders
        # of views or descriptors of the planes drop them when it changes
        self.planes_generation = 0
        self._pending_rebuild_status: torch.Tensor | None = None   # a rebuild's unread errors
        self._append_geo: tuple | None = None     # ma_append_packed's plane geometry (_append_packed)
        self._append_kv: tuple | None = None      # and its new tokens' descriptors
        for name in _UNITS:
            setattr(self, name, None)
        gk = quant.key_token_group
        tokens = min(_ceil_to(self.max_tokens, gk), self._START_TOKENS)
        self._planes = self._plane_specs()
        # bytes of one row (axis 3) of each plane over every layer and lane: the accounting
        # below is arithmetic on the lengths, not tensor slicing
        lanes = self.num_layers * self.batch_size * self.num_kv_heads
        self._row_bytes = {name: lanes * math.prod(row) * torch.empty(0, dtype=dt).element_size()
                           for name, (row, dt) in self._planes.items()}
        self._realloc(tokens=max(tokens, gk), residual=max(1, quant.residual_tokens + gk))

    # -- the plane table ----------------------------------------------------------------------
    def _plane_specs(self) -> dict:
        """name -> (row shape after axis 3, dtype) of every plane this layout stores."""
        q, d = self.quant, self.head_dim
        specs = {}
        if q.k_bits == 16:
            specs["k_fp"] = ((d,), self.compute_dtype)
        else:
            specs["k_q"] = ((d, q.key_token_group * q.k_bits // 8), torch.uint8)
            specs["k_scale"] = specs["k_zero"] = ((d,), self.param_dtype)
            specs["k_residual"] = ((d,), self.compute_dtype)
        if q.v_bits == 16:
            specs["v_fp"] = ((d,), self.compute_dtype)
        else:
            nvg = d // q.value_channel_group
            specs["v_q"] = ((nvg, q.value_channel_group * q.v_bits // 8), torch.uint8)
            specs["v_scale"] = specs["v_zero"] = ((nvg,), self.param_dtype)
            specs["v_residual"] = ((d,), self.compute_dtype)
        return specs

    def _rows_in_use(self, unit: str) -> int:
        gk = self.quant.key_token_group
        if unit == "grp":
            return -(-self.quantized_length // gk)
        if unit == "res":
            return self.residual_length
        if unit == "qtok":
            return self.quantized_length
        return self.length

    def _realloc(self, *, tokens: int | None = None, residual: int | None = None) -> None:
        """Give the token planes room for `tokens` rows (key-group planes tokens / KG) and
        the residual planes room for `residual` rows, keeping the rows in use."""
        lead = (self.num_layers, self.batch_size, self.num_kv_heads)
        gk = self.quant.key_token_group
        want = {"tok": tokens, "qtok": tokens, "grp": None if tokens is None else -(-tokens // gk), "res": residual}
        for name, (row, dtype) in self._planes.items():
            unit = _UNITS[name]
            rows = want[unit]
            if rows is None:
                continue
            new = torch.empty(lead + (rows,) + row, device=self.device, dtype=dtype)
            old = getattr(self, name)
            keep = min(self._rows_in_use(unit), rows) if old is not None else 0
            if keep:
                new[:, :, :, :keep].copy_(old[:, :, :, :keep])
            setattr(self, name, new)
        self.planes_generation += 1

    @property
    def capacity(self) -> int:
        """Token rows allocated (the tokens the store can hold before it grows)."""
        t = self.v_q if self.v_q is not None else self.v_fp
        return int(t.shape[3])

    @property
    def residual_capacity(self) -> int:
        return 0 if self.k_residual is None else int(self.k_residual.shape[3])

    def _reserve(self, tokens: int) -> None:
        """Room for `tokens` stored entries, growing geometrically up to max_tokens."""
        if tokens <= self.capacity:
            return
        if tokens > self.max_tokens:
            raise RuntimeError(f"KV cache capacity exceeded: {tokens}>{self.max_tokens}")
        gk = self.quant.key_token_group
        grown = max(tokens, int(self.capacity * self._GROWTH))
        self._realloc(tokens=min(_ceil_to(grown, gk), _ceil_to(self.max_tokens, gk)))

    def _reserve_residual(self, rows: int) -> None:
        if rows <= self.residual_capacity:
            return
        self._realloc(residual=max(rows, int(self.residual_capacity * self._GROWTH), 64))

    # -- sizes -----------------------------------------------------------------------------
    def __len__(self) -> int:
        return self.num_layers if self.length > 0 else 0

    def get_seq_length(self, layer_idx: int = 0) -> int:
        """Logical length: the next position (stored entries + dropped ones)."""
        return self.length + self.dropped

    def get_max_cache_shape(self) -> int:
        return self.max_tokens

    @property
    def append_in_progress(self) -> bool:
        return self._append_plan is not None

    # -- append protocol ------------------------------------------------------------------
    def reset(self) -> None:
        self.length = self.quantized_length = self.residual_length = self.dropped = 0
        self._append_plan = None

    def begin_append(self, new_tokens: int) -> AppendPlan:
        """Open an append of `new_tokens` to every layer.  A packed store quantizes whole
        key groups of [residual | new] and keeps the rest -- at least residual_tokens, fewer
        than residual_tokens + KG -- as the bf16 residual; in stage mode everything stays bf16."""
        if self._append_plan is not None:
            raise RuntimeError("another cache append is already in progress")
        if new_tokens <= 0:
            raise ValueError("new_tokens must be positive")
        self._reserve(self.length + new_tokens)
        move, tail = 0, 0
        if self.quant.packed:
            tail = self.residual_length + new_tokens
            over = tail - self.quant.residual_tokens
            if over > 0 and not self.stage:
                move = over - over % self.quant.key_token_group
            self._reserve_residual(tail - move + 1)
        plan = AppendPlan(old_length=self.length, new_tokens=int(new_tokens), old_residual=self.residual_length,
                          quantize_from_residual=move, new_residual=tail - move, staged_layers=set())
        self._append_plan = plan
        return plan

    def abort_append(self) -> None:
        self._append_plan = None

    def stage_layer(self, layer_idx: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """Write one layer's new entries: 16-bit planes get them at [length, length + T) by
        the append kernel; packed planes quantize the whole key groups of [residual | new]
        and keep the rest as the residual."""
        plan = self._append_plan
        if plan is None:
            raise RuntimeError("begin_append must be called before stage_layer")
        if layer_idx in plan.staged_layers:
            raise RuntimeError(f"layer {layer_idx} was staged twice")
        expected = (self.batch_size, self.num_kv_heads, plan.new_tokens, self.head_dim)
        if tuple(key.shape) != expected or tuple(value.shape) != expected:
            raise ValueError(f"append tensor shape mismatch: expected {expected}, got K={tuple(key.shape)}, "
                             f"V={tuple(value.shape)}")
        N.require_gpu(key, "key")
        if self.k_fp is not None:
            append_tokens(key, self.k_fp[layer_idx], plan.old_length)
        if self.v_fp is not None:
            append_tokens(value, self.v_fp[layer_idx], plan.old_length)
        if self.quant.packed and self._append_fused(key, value):
            self._append_packed(layer_idx, plan, key, value)
        elif self.quant.packed:
            from .kernels.ops import quantize_key_groups_into, quantize_values_into

            move, keep = plan.quantize_from_residual, plan.new_residual
            k_tail = self._tail(self.k_residual[layer_idx], plan.old_residual, key)
            v_tail = self._tail(self.v_residual[layer_idx], plan.old_residual, value)
            if move:
                gk = self.quant.key_token_group
                g0, t0 = self.quantized_length // gk, self.quantized_length
                gsl, tsl = slice(g0, g0 + move // gk), slice(t0, t0 + move)
                quantize_key_groups_into(k_tail[:, :, :move].contiguous(), self.k_q[layer_idx, :, :, gsl],
                                         self.k_scale[layer_idx, :, :, gsl], self.k_zero[layer_idx, :, :, gsl],
                                         bits=self.quant.k_bits, token_group=gk, backend=self.backend)
                quantize_values_into(v_tail[:, :, :move].contiguous(), self.v_q[layer_idx, :, :, tsl],
                                     self.v_scale[layer_idx, :, :, tsl], self.v_zero[layer_idx, :, :, tsl],
                                     bits=self.quant.v_bits, channel_group=self.quant.value_channel_group,
                                     backend=self.backend)
            if keep:
                append_tokens(k_tail[:, :, move:], self.k_residual[layer_idx], 0)
                append_tokens(v_tail[:, :, move:], self.v_residual[layer_idx], 0)
        plan.staged_layers.add(layer_idx)

    def _append_fused(self, key: torch.Tensor, value: torch.Tensor) -> bool:
        """Whether ma_append_packed serves this append: new tokens in the compute dtype (so
        [residual | new] needs no conversion), the built 4-bit widths and groups."""
        q = self.quant
        return (key.dtype == self.compute_dtype and value.dtype == self.compute_dtype and key.stride(-1) == 1
                and value.stride(-1) == 1 and q.k_bits == 4 and q.v_bits == 4 and q.key_token_group == 32
                and q.value_channel_group == 32 and self.k_fp is None and self.v_fp is None)

    _APPEND_PLANES = ("k_q", "k_scale", "k_zero", "v_q", "v_scale", "v_zero", "k_residual", "v_residual")

    def _append_packed(self, layer_idx: int, plan: "AppendPlan", key: torch.Tensor, value: torch.Tensor) -> None:
        """One layer's packed append in one ma_append_packed call: the whole key groups of
        [residual | new] quantized into the planes after the quantized part, the rest left
        as the residual (the same bytes as the quantizers over the concatenated tail).  The
        planes' strides and element sizes are kept while the planes are the same storage,
        so a call computes only its addresses."""
        move, keep = plan.quantize_from_residual, plan.new_residual
        planes = [getattr(self, name) for name in self._APPEND_PLANES]
        # every replacement of the planes bumps planes_generation (a new plane may reuse a
        # freed one's address with other strides)
        ptrs = (self.planes_generation,) + tuple(t.data_ptr() for t in planes)
        geo = self._append_geo
        if geo is None or geo[0] != ptrs:
            # per plane: (base address, bytes per layer, bytes per row unit) and the strides of
            # a layer's view; the residual planes as ma_tensor4 templates
            lay = [(t.data_ptr(), t.stride(0) * t.element_size(), t.stride(3) * t.element_size()) for t in planes]
            arrs = [N.i64arr(*t.stride()[1:5]) for t in planes[0:1]] + [N.i64arr(*planes[1].stride()[1:4])] + \
                [N.i64arr(*planes[3].stride()[1:5])] + [N.i64arr(*planes[4].stride()[1:4])]
            kres, vres = N.t4(planes[6][0]), N.t4(planes[7][0])
            geo = self._append_geo = (ptrs, lay, arrs, kres, vres)
        _, lay, arrs, kres, vres = geo
        g0, t0 = self.quantized_length // self.quant.key_token_group, self.quantized_length

        def at(i, row):
            base, per_layer, per_row = lay[i]
            return base + layer_idx * per_layer + row * per_row

        kres.ptr, vres.ptr = at(6, 0), at(7, 0)
        # the new tokens' descriptors are kept while their geometry is the same (a decode
        # loop stages same-shaped blocks): only the two addresses change
        kv = (key.shape, key.stride(), key.dtype, value.stride(), value.dtype)
        hit = self._append_kv
        if hit is None or hit[0] != kv:
            hit = self._append_kv = (kv, N.t4(key), N.t4(value), N.load().ma_append_packed)
        _, kt, vt, fn = hit
        kt.ptr, vt.ptr = key.data_ptr(), value.data_ptr()
        b, h, t, d = kv[0]
        N.check(fn(kres, vres, plan.old_residual, kt, vt, b, h, t, d, move, keep, at(0, g0), arrs[0], at(1, g0),
                   at(2, g0), arrs[1], at(3, t0), arrs[2], at(4, t0), at(5, t0), arrs[3], N.stream_of(key)),
                "ma_append_packed")

    def _tail(self, residual: torch.Tensor, old: int, new: torch.Tensor) -> torch.Tensor:
        """[residual rows 0..old | new] as one compute-dtype tensor (a copy when old > 0)."""
        if not old:
            return new.to(self.compute_dtype)
        b, h, t, d = new.shape
        out = torch.empty((b, h, old + t, d), device=self.device, dtype=self.compute_dtype)
        append_tokens(residual[:, :, :old], out, 0)
        append_tokens(new, out, old)
        return out

    def commit_append(self) -> None:
        plan = self._append_plan
        if plan is None:
            raise RuntimeError("no append is in progress")
        missing = set(range(self.num_layers)) - plan.staged_layers
        if missing:
            raise RuntimeError(f"cannot commit: layers not staged: {sorted(missing)}")
        self.length += plan.new_tokens
        if self.quant.packed:
            self.quantized_length += plan.quantize_from_residual
            self.residual_length = plan.new_residual
            assert self.quantized_length + self.residual_length == self.length, "cache length invariant failed"
        self._append_plan = None
        self._note_peak()

    def load_dynamic_cache(self, dynamic_cache) -> None:
        """Fill an empty cache with a prefill's per-layer K / V (the reference's
        load_dynamic_cache, cache.py:568-606): one append of get_seq_length() tokens, each
        layer staged through the HIP append and quantizers; any failure aborts the append.
        A layer is read by whichever access the object offers: ``cache[i]`` -> (K, V), the
        ``key_cache`` / ``value_cache`` lists, or ``layers[i].keys`` / ``.values``."""
        if self.length != 0 or self._append_plan is not None:
            raise RuntimeError("load_dynamic_cache requires an empty cache")
        if dynamic_cache is None:
            return
        n = int(dynamic_cache.get_seq_length())
        if n == 0:
            return
        if n > self.max_tokens:
            raise RuntimeError(f"prefill cache length {n} exceeds capacity {self.max_tokens}")
        self.begin_append(n)
        try:
            for layer in range(self.num_layers):
                key, value = _dynamic_layer(dynamic_cache, layer)
                self.stage_layer(layer, key[..., :n, :].contiguous(), value[..., :n, :].contiguous())
            self.commit_append()
        except BaseException:
            self.abort_append()
            raise

    # -- views ----------------------------------------------------------------------------
    def layer_view(self, layer_idx: int) -> LayerCacheView:
        """The stored prefix of one layer: every plane cut to its rows in use (views)."""
        if not 0 <= layer_idx < self.num_layers:
            raise IndexError(layer_idx)
        cut = {name: None if getattr(self, name) is None
               else getattr(self, name)[layer_idx, :, :, :self._rows_in_use(_UNITS[name])] for name in _UNITS}
        return LayerCacheView(
            k_bits=self.quant.k_bits, v_bits=self.quant.v_bits, length=self.length,
            quantized_length=self.quantized_length, residual_length=self.residual_length,
            key_token_group=self.quant.key_token_group, value_channel_group=self.quant.value_channel_group,
            head_dim=self.head_dim, key_mode=self.quant.key_mode, k_chan=None, **cut)

    def all_layers_view(self) -> LayerCacheView:
        """Every layer's stored prefix as one view with the layers folded into the batch axis
        ([L * B, H, rows, ...] planes, rows in use), for kernels that treat every (layer,
        batch, KV head) lane alike."""
        cut = {name: None if getattr(self, name) is None
               else getattr(self, name)[:, :, :, :self._rows_in_use(_UNITS[name])].flatten(0, 1) for name in _UNITS}
        return LayerCacheView(
            k_bits=self.quant.k_bits, v_bits=self.quant.v_bits, length=self.length,
            quantized_length=self.quantized_length, residual_length=self.residual_length,
            key_token_group=self.quant.key_token_group, value_channel_group=self.quant.value_channel_group,
            head_dim=self.head_dim, key_mode=self.quant.key_mode, k_chan=None, **cut)

    def dequantize_layer(self, layer_idx: int, *, dtype: torch.dtype | None = None):
        """One layer's whole stored prefix as [B, H, length, D] K and V (ma_dequant_prefix)."""
        from .kernels.splitk import Prefix, dequantize_prefix

        return dequantize_prefix(Prefix.from_view(self.layer_view(layer_idx)), self.batch_size, self.num_kv_heads,
                                 self.head_dim, dtype=dtype or self.compute_dtype)

    def gather_layer_reference(self, layer_idx: int, indices: torch.Tensor, *, dtype: torch.dtype | None = None):
        """Stored entries indices [B, H, k] of one layer, dequantized (ma_gather_kv)."""
        from .kernels.ops import gather_packed_kv

        return gather_packed_kv(self.layer_view(layer_idx), indices, dtype=dtype or self.compute_dtype)

    # -- compaction -------------------------------------------------------------------------
    def _check_keep(self, keep: torch.Tensor) -> int:
        if self._append_plan is not None:
            raise RuntimeError("compaction during an append")
        if tuple(keep.shape[:3]) != (self.num_layers, self.batch_size, self.num_kv_heads) or keep.dim() != 4:
            raise ValueError(f"keep must be [L, B, Hkv, C], got {tuple(keep.shape)}")
        c = int(keep.shape[-1])
        if c > self.length:
            raise ValueError("compact cannot grow the cache")
        return c

    def _sparse_after(self, c: int) -> bool:
        """Whether storage holding c entries is mostly empty (then it is given back)."""
        return self.capacity > 2 * c + 2048

    def _shrink_if_sparse(self, c: int) -> None:
        """Give back storage when a compaction left it mostly empty."""
        if self._sparse_after(c):
            self._realloc(tokens=_ceil_to(c + 1024, self.quant.key_token_group))

    def _gather_into_smaller(self, keep2: torch.Tensor, c: int) -> None:
        """A 16-bit store's compaction that leaves it mostly empty: the kept rows (keep2
        [L * B, H, c]) gathered by ma_gather_kv straight into smaller planes, one read and
        one write of each kept row, instead of moving them in place and copying them again
        into smaller planes.  Every row is copied exactly (16-bit values through f32)."""
        from .kernels.ops import gather_packed_kv
        from .kernels.splitk import Prefix

        lb, h, d = self.num_layers * self.batch_size, self.num_kv_heads, self.head_dim
        rows = _ceil_to(c + 1024, self.quant.key_token_group)
        old_k, old_v = self.k_fp, self.v_fp
        src = Prefix.dense(old_k.view(lb, h, old_k.shape[3], d)[:, :, :self.length],
                           old_v.view(lb, h, old_v.shape[3], d)[:, :, :self.length])
        new_k = torch.empty((self.num_layers, self.batch_size, h, rows, d), device=self.device, dtype=old_k.dtype)
        new_v = torch.empty_like(new_k, dtype=old_v.dtype)
        gather_packed_kv(src, keep2, out_key=new_k.view(lb, h, rows, d)[:, :, :c],
                         out_value=new_v.view(lb, h, rows, d)[:, :, :c])
        self.k_fp, self.v_fp = new_k, new_v
        self.planes_generation += 1
        self.length = c

    def compact(self, keep: torch.Tensor) -> None:
        """Keep only stored entries keep[l, b, h, :] of every layer, in that order; positions
        are unchanged (dropped grows by the entries removed).  16-bit planes move in place
        (one ma_compact_tokens call over every layer); a packed store gathers the survivors
        dequantized and appends them again, so they are quantized afresh."""
        from .kernels.ops import gather_packed_kv

        c = self._check_keep(keep)
        removed = self.length - c
        if not self.quant.packed:
            lb, h = self.num_layers * self.batch_size, self.num_kv_heads
            if self._sparse_after(c):
                self._gather_into_smaller(keep.reshape(lb, h, c), c)
            else:
                planes = [t.view(lb, h, t.shape[3], t.shape[4]) for t in (self.k_fp, self.v_fp)]
                compact_tokens(planes, keep.reshape(lb, h, c), self.length)
                self.length = c
        else:
            kv = [gather_packed_kv(self.layer_view(layer), keep[layer].to(torch.int64), dtype=self.compute_dtype)
                  for layer in range(self.num_layers)]
            self.length = self.quantized_length = self.residual_length = 0
            self._shrink_if_sparse(c)
            self.begin_append(c)
            for layer, (k, v) in enumerate(kv):
                self.stage_layer(layer, k, v)
            self.commit_append()
        self.dropped += removed
        self._note_peak()

    def compact_tokens(self, keep: torch.Tensor) -> None:
        """Keep stored entries keep[l, b, h, :] by moving their rows, exact for per-token
        planes (16-bit K/V, per-token packed values).  Keys packed per channel over token
        groups cannot move token by token: ValueError."""
        if self.k_q is not None:
            raise ValueError("compact_tokens: keys packed per channel over token groups cannot be moved per token")
        if self.residual_length:
            raise RuntimeError("compact_tokens needs a fully quantized cache")
        c = self._check_keep(keep)
        lb, h = self.num_layers * self.batch_size, self.num_kv_heads
        planes = [getattr(self, name).view(lb, h, *getattr(self, name).shape[3:])
                  for name in ("v_q", "v_scale", "v_zero", "k_fp", "v_fp") if getattr(self, name) is not None]
        compact_tokens(planes, keep.reshape(lb, h, c), self.length)
        self.dropped += self.length - c
        self.length = c
        self.quantized_length = c if self.quant.packed else 0
        self._shrink_if_sparse(c)
        self._note_peak()

    # -- packed eviction rebuild ------------------------------------------------------------
    def rebuild(self, groups_before: torch.Tensor, encode: torch.Tensor, groups_after: torch.Tensor,
                stage: torch.Tensor) -> torch.Tensor:
        """The reference's PackedKVCache.rebuild contract (cache.py:236-335): new storage
        [groups_before | encode, quantized | groups_after] + stage as the bf16 residual.
        Index tensors [L, B, H, n] int64, -1-padded: groups_* old key groups copied as they
        are (-1: a copy of group 0, to be masked), encode old slots quantized into fresh
        groups (-1: zeros), stage old slots kept bf16 (-1: zeros).  Returns the remap
        [L, B, H, old length]: the new slot of every old slot, -1 if dropped."""
        return self._rebuild(groups_before, encode, groups_after, stage)

    def check_rebuild(self) -> None:
        """Raise the errors of a rebuild run with check=False (see _rebuild), if any; one
        small copy to the host.  A no-op when none is pending."""
        from .kernels.rebuild import raise_rebuild_status

        status, self._pending_rebuild_status = self._pending_rebuild_status, None
        if status is not None:
            raise_rebuild_status(status)

    def _rebuild(self, groups_before, encode, groups_after, stage, phys: torch.Tensor | None = None,
                 live: int = 0, check: bool = True) -> torch.Tensor:
        """rebuild(), with the eviction state's slots phys (int32 [L, B, H, capacity]) rewritten
        through the remap in the same launch.  New planes are allocated and written by
        ma_rebuild_packed over every layer at once (the lanes of all layers folded into the
        batch axis); the old ones are dropped.  check=False leaves the launch's error status
        on the device, to be raised by check_rebuild() -- called by the next rebuild -- instead
        of reading it back now."""
        from .kernels.rebuild import rebuild_packed

        self.check_rebuild()

        if self._append_plan is not None:
            raise RuntimeError("rebuild during an append")
        if self.k_q is None or self.v_q is None:
            raise ValueError("rebuild needs a packed (k_bits, v_bits < 16) cache")
        if self.quant.k_bits != 4 or self.quant.v_bits != 4 or self.k_scale.dtype != torch.float16:
            raise KernelUnavailableError("the packed rebuild is built for 4-bit codes with float16 scale / zero")
        lead = (self.num_layers, self.batch_size, self.num_kv_heads)
        lists = {"groups_before": groups_before, "encode": encode, "groups_after": groups_after, "stage": stage}
        for name, t in lists.items():
            if t.dim() != 4 or tuple(t.shape[:3]) != lead:
                raise ValueError(f"{name} must be [L, B, H, n], got {tuple(t.shape)}")
        gk = self.quant.key_token_group
        groups = groups_before.shape[-1] + -(-encode.shape[-1] // gk) + groups_after.shape[-1]
        ql, st = groups * gk, stage.shape[-1]
        old_planes = {name: getattr(self, name) for name in self._planes}
        old_len, old_q, old_r = self.length, self.quantized_length, self.residual_length
        # fresh planes sized for the new layout (and room to append), written by the kernel
        for name in self._planes:
            setattr(self, name, None)
        self.length = self.quantized_length = self.residual_length = 0
        self._realloc(tokens=_ceil_to(ql + st + 1024, gk), residual=max(st + 256, 64))
        remap = torch.empty(lead + (old_len,), device=self.device, dtype=torch.int64)

        new_planes = {name: getattr(self, name) for name in self._planes}
        status = rebuild_packed(self._folded_native(old_planes, old_q, old_r), self._folded_native(new_planes, ql, st),
                                B=lead[0] * lead[1],
                                H=lead[2], D=self.head_dim, groups_before=groups_before, encode=encode,
                                groups_after=groups_after, stage=stage, remap=remap, phys=phys, live=live,
                                check=check)
        self._pending_rebuild_status = status
        self.length, self.quantized_length, self.residual_length = ql + st, ql, st
        self.dropped += old_len - self.length
        self._note_peak()
        return remap

    def _folded_native(self, planes: dict, nq: int, nf: int) -> N.MaPrefix:
        """The C-ABI descriptor of whole 4-bit storage planes [L, B, H, ...] with the layers
        folded into the batch axis (lane (l, b, h) = batch row l * B + b), as
        ma_rebuild_packed reads the old storage and writes the new one.  The planes are this
        cache's own allocations (contiguous; 4-bit codes and float16 scale / zero, as _rebuild
        checks first), so the descriptor is filled from their strides without building views."""
        kq, ks, kz, vq, vs, vz, kf, vf = (planes[x] for x in self._APPEND_PLANES)
        p = N.MaPrefix()
        p.nq, p.nf, p.kbits, p.vbits = int(nq), int(nf), 4, 4
        p.kgroup, p.vgroup = self.quant.key_token_group, self.quant.value_channel_group
        p.kq, p.ks, p.kz, p.vq, p.vs, p.vz = (t.data_ptr() for t in (kq, ks, kz, vq, vs, vz))
        p.kf, p.vf = kf.data_ptr(), vf.data_ptr()
        p.fdtype = N.dtype_code(kf.dtype)
        p.skq[:] = kq.stride()[1:5]
        p.svq[:] = vq.stride()[1:5]
        p.sks[:] = ks.stride()[1:4]
        p.svs[:] = vs.stride()[1:4]
        p.skf[:] = kf.stride()[1:4]
        p.svf[:] = vf.stride()[1:4]
        return p

    # -- memory accounting --------------------------------------------------------------------
    def allocated_nbytes(self) -> int:
        """Bytes of every plane as allocated."""
        return int(sum(t.numel() * t.element_size() for t in (getattr(self, n) for n in self._planes)))

    def bf16_equivalent_nbytes(self) -> int:
        """What the logical length would take as bf16 K and V."""
        return 4 * self.num_layers * self.batch_size * self.num_kv_heads * self.head_dim * self.get_seq_length()

    def logical_nbytes(self) -> dict[str, int]:
        """Bytes in use per part (the reference's keys, cache.py:769-811): the rows in use of
        each plane, grouped into payload (codes or 16-bit rows), metadata (scale / zero)
        and residual, for K and for V."""
        part = {"k_q": "key_payload", "k_fp": "key_payload", "k_scale": "key_metadata", "k_zero": "key_metadata",
                "k_residual": "key_residual", "v_q": "value_payload", "v_fp": "value_payload",
                "v_scale": "value_metadata", "v_zero": "value_metadata", "v_residual": "value_residual"}
        out = dict.fromkeys(("key_payload", "key_metadata", "key_residual", "value_payload", "value_metadata",
                             "value_residual"), 0)
        for name in self._planes:
            rows = min(self._rows_in_use(_UNITS[name]), getattr(self, name).shape[3])
            out[part[name]] += rows * self._row_bytes[name]
        out["total"] = sum(out.values())
        return out

    def _note_peak(self) -> None:
        """Track the high-water marks of bytes in use and allocated; with a memory_trace list
        attached, record (next position, in use, allocated) at every change."""
        now = (self.logical_nbytes()["total"], self.allocated_nbytes())
        self.peak_used_bytes, self.peak_allocated_bytes = (max(a, b) for a, b in
                                                           zip((self.peak_used_bytes, self.peak_allocated_bytes), now))
        if self.memory_trace is not None:
            self.memory_trace.append([self.get_seq_length(), *now])
