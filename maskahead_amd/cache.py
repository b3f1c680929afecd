"""Per-layer KV cache of the read/keep path (the reference's ``maskahead.cache``).

``PackedKVCache`` keeps the reference's storage format and bookkeeping (cache.py:37-811):
the same tensors, shapes and capacity-padded layouts, the same append protocol
(begin_append / stage_layer / commit_append), the same logical length with ``dropped``
entries after a compaction, and the same ``layer_view``.  What moves data runs on the
gfx950 kernels: the append of a bf16 block and the residual tail (ma_append_tokens),
the 4-bit quantizers (ma_quantize_keys / ma_quantize_values), the dequant
(ma_dequant_prefix), the gather (ma_gather_kv) and compaction in place
(ma_compact_tokens), where the reference dequantizes every layer, gathers and
re-appends.

Built for 4-bit (key groups of 32 tokens per channel, value groups of 32 channels per
token, f16 scale/zero) and 16-bit layouts; other valid quantization settings raise
KernelUnavailableError.  The packed lazy rebuild (``stage`` / ``rebuild``,
cache.py:236-335) runs in one launch of ma_rebuild_packed over every layer.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _native as N
from ._native import KernelUnavailableError
from .config import QuantizationConfig
from .kernels.keep import append_tokens, compact_tokens


def _dtype_from_name(name: str) -> torch.dtype:
    return {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}[name]


@dataclass(slots=True)
class AppendPlan:
    """cache.py:27-34."""
    old_length: int
    new_tokens: int
    old_residual: int
    quantize_from_residual: int
    new_residual: int
    staged_layers: set[int]


@dataclass(slots=True)
class LayerCacheView:
    """One layer's slice of the cache (cache.py:37-60): views, no copies."""
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


class PackedKVCache:
    """Token storage of every layer: [L, B, Hkv, capacity, ...] tensors (cache.py:63-189)."""

    _TOKEN_AXIS = {"k_fp": 3, "v_fp": 3, "v_q": 3, "v_scale": 3, "v_zero": 3}
    _GROUP_AXIS = {"k_q": 3, "k_scale": 3, "k_zero": 3}

    def __init__(self, *, num_layers: int, batch_size: int, num_kv_heads: int, head_dim: int, max_tokens: int,
                 quant: QuantizationConfig, device: torch.device | str, compute_dtype: torch.dtype = torch.bfloat16,
                 backend: str = "auto") -> None:
        quant.validate(head_dim=head_dim)
        if num_layers <= 0 or batch_size <= 0 or num_kv_heads <= 0 or head_dim <= 0:
            raise ValueError("all cache dimensions must be positive")
        if backend not in ("auto", "triton", "torch", "hip"):
            raise ValueError(f"unknown cache backend: {backend}")
        if backend == "torch":
            raise KernelUnavailableError("backend='torch' is the reference's CPU path; this cache runs on the "
                                         "HIP kernels only")
        quant.require_built()
        self.num_layers = int(num_layers)
        self.batch_size = int(batch_size)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.max_tokens = int(max_tokens)
        self.quant = quant
        self.device = torch.device(device)
        self.compute_dtype = compute_dtype
        self.param_dtype = _dtype_from_name(quant.param_dtype)
        self.backend = backend

        self.length = 0
        self.quantized_length = 0
        self.residual_length = 0
        self._append_plan: AppendPlan | None = None

        gk = quant.key_token_group
        self.capacity = min(self.max_tokens, max(gk, (1024 // gk) * gk))
        self.dropped = 0
        self.stage = False
        self.peak_used_bytes = 0
        self.peak_allocated_bytes = 0
        self.memory_trace: list[list[int]] | None = None
        self.rotation = None
        self.key_center = None
        l, b, h, d, n = self.num_layers, self.batch_size, self.num_kv_heads, self.head_dim, self.capacity
        gv = quant.value_channel_group
        self.residual_capacity = max(1, quant.residual_tokens + gk - 1)

        self.k_chan = None
        self.k_fp = self.v_fp = None
        self.k_q = self.k_scale = self.k_zero = None
        self.v_q = self.v_scale = self.v_zero = None
        self.k_residual = self.v_residual = None
        dev = self.device
        if quant.k_bits == 16:
            self.k_fp = torch.empty((l, b, h, n, d), device=dev, dtype=compute_dtype)
        else:
            groups = math.ceil(n / gk)
            self.k_q = torch.empty((l, b, h, groups, d, gk * quant.k_bits // 8), device=dev, dtype=torch.uint8)
            self.k_scale = torch.empty((l, b, h, groups, d), device=dev, dtype=self.param_dtype)
            self.k_zero = torch.empty_like(self.k_scale)
            self.k_residual = torch.empty((l, b, h, self.residual_capacity, d), device=dev, dtype=compute_dtype)
        if quant.v_bits == 16:
            self.v_fp = torch.empty((l, b, h, n, d), device=dev, dtype=compute_dtype)
        else:
            self.v_q = torch.empty((l, b, h, n, d // gv, gv * quant.v_bits // 8), device=dev, dtype=torch.uint8)
            self.v_scale = torch.empty((l, b, h, n, d // gv), device=dev, dtype=self.param_dtype)
            self.v_zero = torch.empty_like(self.v_scale)
            self.v_residual = torch.empty((l, b, h, self.residual_capacity, d), device=dev, dtype=compute_dtype)

    # -- sizes -----------------------------------------------------------------------------
    def __len__(self) -> int:
        return self.num_layers if self.length > 0 else 0

    def get_seq_length(self, layer_idx: int = 0) -> int:
        """Logical length (next position); physical storage holds self.length entries."""
        return self.length + self.dropped

    def get_max_cache_shape(self) -> int:
        return self.max_tokens

    @property
    def append_in_progress(self) -> bool:
        return self._append_plan is not None

    # -- storage growth (cache.py:223-340) -------------------------------------------------
    def _resize(self, cap: int) -> None:
        """Reallocate token storage to cap tokens, keeping the first self.length."""
        gk = self.quant.key_token_group
        cap = min(self.max_tokens, -(-cap // gk) * gk)
        keep_t, keep_g = self.length, -(-self.quantized_length // gk)
        for name, axis in list(self._TOKEN_AXIS.items()) + list(self._GROUP_AXIS.items()):
            old = getattr(self, name)
            if old is None:
                continue
            shape = list(old.shape)
            is_group = name in self._GROUP_AXIS
            shape[axis] = -(-cap // gk) if is_group else cap
            new = torch.empty(shape, device=old.device, dtype=old.dtype)
            n = keep_g if is_group else keep_t
            if n:
                new.narrow(axis, 0, n).copy_(old.narrow(axis, 0, n))
            setattr(self, name, new)
        self.capacity = cap

    def _grow_residual(self, needed: int) -> None:
        cap = max(needed, int(self.residual_capacity * 1.5), 64)
        for name in ("k_residual", "v_residual"):
            old = getattr(self, name)
            if old is None:
                continue
            shape = list(old.shape)
            shape[3] = cap
            new = torch.empty(shape, device=old.device, dtype=old.dtype)
            if self.residual_length:
                new[:, :, :, :self.residual_length].copy_(old[:, :, :, :self.residual_length])
            setattr(self, name, new)
        self.residual_capacity = cap

    def _grow(self, needed: int) -> None:
        if needed > self.max_tokens:
            raise RuntimeError(f"KV cache capacity exceeded: {needed}>{self.max_tokens}")
        self._resize(max(needed, int(self.capacity * 1.5)))

    # -- append protocol (cache.py:370-566) ------------------------------------------------
    def reset(self) -> None:
        self.dropped = 0
        self.length = 0
        self.quantized_length = 0
        self.residual_length = 0
        self._append_plan = None

    def begin_append(self, new_tokens: int) -> AppendPlan:
        if self._append_plan is not None:
            raise RuntimeError("another cache append is already in progress")
        if new_tokens <= 0:
            raise ValueError("new_tokens must be positive")
        if self.length + new_tokens > self.capacity:
            self._grow(self.length + new_tokens)
        if not self.quant.packed:
            move = new_residual = 0
        else:
            total_tail = self.residual_length + new_tokens
            if self.stage:
                move = 0
            else:
                excess = max(0, total_tail - self.quant.residual_tokens)
                move = (excess // self.quant.key_token_group) * self.quant.key_token_group
            new_residual = total_tail - move
            if new_residual >= self.residual_capacity:
                self._grow_residual(new_residual + 1)
        plan = AppendPlan(old_length=self.length, new_tokens=int(new_tokens), old_residual=self.residual_length,
                          quantize_from_residual=move, new_residual=new_residual, staged_layers=set())
        self._append_plan = plan
        return plan

    def abort_append(self) -> None:
        self._append_plan = None

    def stage_layer(self, layer_idx: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """Write one layer's new entries: bf16 layouts by the append kernel at
        [length, length + T); packed layouts quantize whole key groups out of
        [residual | new] and keep the rest as the bf16 residual (cache.py:423-547)."""
        from .kernels.ops import quantize_key_groups_into, quantize_values_into

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
        start = plan.old_length
        if self.quant.k_bits == 16:
            append_tokens(key, self.k_fp[layer_idx], start)
        if self.quant.v_bits == 16:
            append_tokens(value, self.v_fp[layer_idx], start)
        if self.quant.packed:
            old_r, move, remain = plan.old_residual, plan.quantize_from_residual, plan.new_residual
            tails = []
            for src, res in ((key, self.k_residual), (value, self.v_residual)):
                if old_r:
                    tail = torch.empty((self.batch_size, self.num_kv_heads, old_r + plan.new_tokens,
                                        self.head_dim), device=self.device, dtype=self.compute_dtype)
                    append_tokens(res[layer_idx, :, :, :old_r], tail, 0)
                    append_tokens(src, tail, old_r)
                else:
                    tail = src.to(self.compute_dtype)
                tails.append(tail)
            k_tail, v_tail = tails
            if move:
                g0 = self.quantized_length // self.quant.key_token_group
                gc = move // self.quant.key_token_group
                quantize_key_groups_into(k_tail[:, :, :move].contiguous(), self.k_q[layer_idx, :, :, g0:g0 + gc],
                                         self.k_scale[layer_idx, :, :, g0:g0 + gc],
                                         self.k_zero[layer_idx, :, :, g0:g0 + gc], bits=self.quant.k_bits,
                                         token_group=self.quant.key_token_group, backend=self.backend)
                t0 = self.quantized_length
                quantize_values_into(v_tail[:, :, :move].contiguous(), self.v_q[layer_idx, :, :, t0:t0 + move],
                                     self.v_scale[layer_idx, :, :, t0:t0 + move],
                                     self.v_zero[layer_idx, :, :, t0:t0 + move], bits=self.quant.v_bits,
                                     channel_group=self.quant.value_channel_group, backend=self.backend)
            if remain:
                append_tokens(k_tail[:, :, move:], self.k_residual[layer_idx], 0)
                append_tokens(v_tail[:, :, move:], self.v_residual[layer_idx], 0)
        plan.staged_layers.add(layer_idx)

    def commit_append(self) -> None:
        plan = self._append_plan
        if plan is None:
            raise RuntimeError("no append is in progress")
        expected = set(range(self.num_layers))
        if plan.staged_layers != expected:
            raise RuntimeError(f"cannot commit: layers not staged: {sorted(expected - plan.staged_layers)}")
        self.length += plan.new_tokens
        if self.quant.packed:
            self.quantized_length += plan.quantize_from_residual
            self.residual_length = plan.new_residual
        self._append_plan = None
        self._note_peak()
        if self.quant.packed and self.quantized_length + self.residual_length != self.length:
            raise AssertionError("cache length invariant failed")

    # -- views ---------------------------------------------------------------------------
    def layer_view(self, layer_idx: int) -> LayerCacheView:
        """cache.py:608-657."""
        if not 0 <= layer_idx < self.num_layers:
            raise IndexError(layer_idx)
        qg = self.quantized_length // self.quant.key_token_group
        qn, n, rn = self.quantized_length, self.length, self.residual_length

        def cut(t, axis_len):
            return None if t is None else t[layer_idx, :, :, :axis_len]

        return LayerCacheView(
            k_bits=self.quant.k_bits, v_bits=self.quant.v_bits, length=n, quantized_length=qn,
            residual_length=rn, key_token_group=self.quant.key_token_group,
            value_channel_group=self.quant.value_channel_group,
            k_q=cut(self.k_q, qg), k_scale=cut(self.k_scale, qg), k_zero=cut(self.k_zero, qg),
            v_q=cut(self.v_q, qn), v_scale=cut(self.v_scale, qn), v_zero=cut(self.v_zero, qn),
            k_fp=cut(self.k_fp, n), v_fp=cut(self.v_fp, n),
            k_residual=cut(self.k_residual, rn), v_residual=cut(self.v_residual, rn),
            head_dim=self.head_dim, key_mode=self.quant.key_mode, k_chan=None)

    def dequantize_layer(self, layer_idx: int, *, dtype: torch.dtype | None = None):
        """The layer's whole prefix as [B, H, length, D] K and V (cache.py:680-741)."""
        from .kernels.splitk import Prefix, dequantize_prefix

        dtype = dtype or self.compute_dtype
        return dequantize_prefix(Prefix.from_view(self.layer_view(layer_idx)), self.batch_size, self.num_kv_heads,
                                 self.head_dim, dtype=dtype)

    def gather_layer_reference(self, layer_idx: int, indices: torch.Tensor, *, dtype: torch.dtype | None = None):
        """Entries indices [B, H, k] of one layer, dequantized (cache.py:743-751)."""
        from .kernels.ops import gather_packed_kv

        return gather_packed_kv(self.layer_view(layer_idx), indices, dtype=dtype or self.compute_dtype)

    # -- eviction (cache.py:342-367, 659-678) ----------------------------------------------
    def compact(self, keep: torch.Tensor) -> None:
        """Keep only entries keep[l, b, h, :] (physical indices) of every layer, in that
        order; logical positions are unchanged (dropped grows).  16-bit caches are
        compacted in place by one kernel pair over all layers; a packed cache gathers
        the survivors dequantized and re-appends them, as the reference does."""
        from .kernels.ops import gather_packed_kv

        if self._append_plan is not None:
            raise RuntimeError("compact during an append")
        c = int(keep.shape[-1])
        old = self.length
        if c > old:
            raise ValueError("compact cannot grow the cache")
        if tuple(keep.shape[:3]) != (self.num_layers, self.batch_size, self.num_kv_heads):
            raise ValueError(f"keep must be [L, B, Hkv, C], got {tuple(keep.shape)}")
        gk = self.quant.key_token_group
        if not self.quant.packed:
            lb, h = self.num_layers * self.batch_size, self.num_kv_heads
            planes = [t.view(lb, h, t.shape[3], t.shape[4]) for t in (self.k_fp, self.v_fp)]
            compact_tokens(planes, keep.reshape(lb, h, c), old)
            self.length = c
            if self.capacity > 2 * max(c, gk) + 1024:
                self._resize(c + 1024)
            self.dropped += old - c
            self._note_peak()
            return
        survivors = [gather_packed_kv(self.layer_view(l), keep[l].to(torch.int64), dtype=self.compute_dtype)
                     for l in range(self.num_layers)]
        self.length = self.quantized_length = self.residual_length = 0
        if self.capacity > 2 * max(c, gk) + 1024:
            self._resize(c + 1024)
        self.begin_append(c)
        for layer_idx, (k, v) in enumerate(survivors):
            self.stage_layer(layer_idx, k, v)
        self.commit_append()
        self.dropped += old - c

    def compact_tokens(self, keep: torch.Tensor) -> None:
        """Keep entries keep[l, b, h, :] by moving their stored rows, exact for per-token
        layouts (cache.py:659-678): 16-bit K/V and per-token packed values.  Packed keys
        grouped over tokens cannot be moved token by token and raise ValueError."""
        if self._append_plan is not None or self.residual_length:
            raise RuntimeError("compact_tokens needs a fully quantized cache")
        if self.k_q is not None:
            raise ValueError("compact_tokens: keys packed per channel over token groups cannot be moved per token")
        c = int(keep.shape[-1])
        lb, h = self.num_layers * self.batch_size, self.num_kv_heads
        planes = []
        for name in ("v_q", "v_scale", "v_zero", "k_fp", "v_fp"):
            t = getattr(self, name)
            if t is not None:
                planes.append(t.view(lb, h, *t.shape[3:]))
        compact_tokens(planes, keep.reshape(lb, h, c), self.length)
        old = self.length
        self.length = c
        self.quantized_length = c if self.quant.packed else 0
        self.dropped += old - c
        if self.capacity > 2 * c + 2048:
            self._resize(c + 1024)
        self._note_peak()

    # -- packed eviction rebuild (cache.py:236-335) ----------------------------------------
    def _fold(self, t: torch.Tensor | None) -> torch.Tensor | None:
        """[L, B, H, ...] storage -> [L*B, H, ...] view: every layer in one launch."""
        return None if t is None else t.flatten(0, 1)

    def rebuild(self, groups_before: torch.Tensor, encode: torch.Tensor, groups_after: torch.Tensor,
                stage: torch.Tensor) -> torch.Tensor:
        """New physical layout [groups_before | encoded | groups_after] + bf16 staging
        (cache.py:236-335).  Index tensors [L, B, H, n] int64, padded with -1:
        groups_before / groups_after old key groups copied bit-exactly (a -1 entry holds a
        copy of group 0 and must be masked by the caller), encode old slots quantized into
        fresh groups, stage old slots kept in bf16 (the new residual; -1: zeros).  Returns
        remap [L, B, H, old_length]: the new slot of every old slot, -1 if dropped."""
        return self._rebuild(groups_before, encode, groups_after, stage)

    def _rebuild(self, groups_before, encode, groups_after, stage, phys: torch.Tensor | None = None,
                 live: int = 0) -> torch.Tensor:
        """rebuild(); phys (the eviction state's int32 [L, B, H, capacity] slots) is
        rewritten through the remap in the same launch (session.py:352-355)."""
        from .kernels.rebuild import rebuild_packed
        from .kernels.splitk import Prefix

        if self._append_plan is not None:
            raise RuntimeError("rebuild during an append")
        if self.k_q is None or self.v_q is None:
            raise ValueError("rebuild needs a packed (k_bits, v_bits < 16) cache")
        gk = self.quant.key_token_group
        L, B, H, D = self.num_layers, self.batch_size, self.num_kv_heads, self.head_dim
        lead = (L, B, H)
        for name, t in (("groups_before", groups_before), ("encode", encode), ("groups_after", groups_after),
                        ("stage", stage)):
            if t.dim() != 4 or tuple(t.shape[:3]) != lead:
                raise ValueError(f"{name} must be [L, B, H, n], got {tuple(t.shape)}")
        dev = self.device
        old_len, old_q, old_r = self.length, self.quantized_length, self.residual_length
        g1, m, g3, st = groups_before.shape[-1], encode.shape[-1], groups_after.shape[-1], stage.shape[-1]
        g2 = -(-m // gk)
        ql = (g1 + g2 + g3) * gk
        new_len = ql + st
        cap = new_len + 1024
        ng_cap = -(-cap // gk)
        kq = torch.empty((L, B, H, ng_cap, D, self.k_q.shape[-1]), device=dev, dtype=self.k_q.dtype)
        ks = torch.empty((L, B, H, ng_cap, D), device=dev, dtype=self.k_scale.dtype)
        kz = torch.empty_like(ks)
        vq = torch.empty((L, B, H, cap, *self.v_q.shape[4:]), device=dev, dtype=self.v_q.dtype)
        vs = torch.empty((L, B, H, cap, self.v_scale.shape[-1]), device=dev, dtype=self.v_scale.dtype)
        vz = torch.empty_like(vs)
        rcap = max(st + 256, 64)
        kr = torch.empty((L, B, H, rcap, D), device=dev, dtype=self.k_residual.dtype)
        vr = torch.empty_like(kr)
        remap = torch.empty((L, B, H, old_len), device=dev, dtype=torch.int64)
        f = self._fold
        old = Prefix(kq=f(self.k_q), ks=f(self.k_scale), kz=f(self.k_zero), vq=f(self.v_q), vs=f(self.v_scale),
                     vz=f(self.v_zero), kf=f(self.k_residual), vf=f(self.v_residual), nq=old_q, nf=old_r,
                     kb=4, vb=4)
        new = Prefix(kq=f(kq), ks=f(ks), kz=f(kz), vq=f(vq), vs=f(vs), vz=f(vz), kf=f(kr), vf=f(vr), nq=ql, nf=st,
                     kb=4, vb=4)
        rebuild_packed(old, new, B=L * B, H=H, D=D, groups_before=groups_before, encode=encode,
                       groups_after=groups_after, stage=stage, remap=remap, phys=phys, live=live)
        self.k_q, self.k_scale, self.k_zero, self.v_q, self.v_scale, self.v_zero = kq, ks, kz, vq, vs, vz
        self.k_residual, self.v_residual = kr, vr
        self.capacity, self.residual_capacity = cap, rcap
        self.length, self.quantized_length, self.residual_length = new_len, ql, st
        self.dropped += old_len - new_len
        self._note_peak()
        return remap

    # -- memory accounting (cache.py:753-811) ----------------------------------------------
    def allocated_nbytes(self) -> int:
        names = ("k_fp", "v_fp", "k_q", "k_scale", "k_zero", "v_q", "v_scale", "v_zero", "k_residual", "v_residual")
        return int(sum(t.numel() * t.element_size() for t in (getattr(self, x) for x in names) if t is not None))

    def bf16_equivalent_nbytes(self) -> int:
        return 2 * 2 * self.num_layers * self.batch_size * self.num_kv_heads * self.head_dim * self.get_seq_length()

    def logical_nbytes(self) -> dict[str, int]:
        l, b, h, d = self.num_layers, self.batch_size, self.num_kv_heads, self.head_dim
        qn, rn = self.quantized_length, self.residual_length
        ps = torch.tensor([], dtype=self.param_dtype).element_size()
        cs = torch.tensor([], dtype=self.compute_dtype).element_size()
        if self.quant.k_bits == 16:
            k_payload, k_meta, k_res = l * b * h * self.length * d * cs, 0, 0
        else:
            k_payload = l * b * h * qn * d * self.quant.k_bits // 8
            k_meta = l * b * h * (qn // self.quant.key_token_group) * d * 2 * ps
            k_res = l * b * h * rn * d * cs
        if self.quant.v_bits == 16:
            v_payload, v_meta, v_res = l * b * h * self.length * d * cs, 0, 0
        else:
            v_payload = l * b * h * qn * d * self.quant.v_bits // 8
            v_meta = l * b * h * qn * (d // self.quant.value_channel_group) * 2 * ps
            v_res = l * b * h * rn * d * cs
        out = {"key_payload": int(k_payload), "key_metadata": int(k_meta), "key_residual": int(k_res),
               "value_payload": int(v_payload), "value_metadata": int(v_meta), "value_residual": int(v_res)}
        out["total"] = sum(out.values())
        return out

    def _note_peak(self) -> None:
        used, alloc = self.logical_nbytes()["total"], self.allocated_nbytes()
        self.peak_used_bytes = max(self.peak_used_bytes, used)
        self.peak_allocated_bytes = max(self.peak_allocated_bytes, alloc)
        if self.memory_trace is not None:
            self.memory_trace.append([self.get_seq_length(), used, alloc])
