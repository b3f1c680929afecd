"""The fast path of a batch of sequences that each have their own cache (ragged prefixes).

The reference session keeps one compact buffer per layer for its whole batch,
``CompactLayerState.key / value`` of [B, Hkv, k + block, D] (session.py:430-454), and
attends every denoising sub-step of a sparse layer over it in one call
(``_compact_attention``, session.py:1286-1336).  ``BatchFastPath`` does the same for
sequences whose prefixes live in caches of their own (so need no padding to the longest):

  * step 0 of a layer runs per sequence, over that sequence's own prefix
    (``FastLayerPath.step0``: split-K attention, value-aware scores, read-set top-k), and
    gathers each read set into that sequence's rows of the layer's shared compact buffer;
  * every later sub-step of a sparse layer is ONE split-K call over the whole batch:
    [B rows of the compact buffer | the block], the queries and block K/V as the batched
    forward hands them over ([B, H, T, D]);
  * dense layers (below ``dense_prefix_layers``, or with no read set) attend each
    sequence's live prefix, per sequence.

The read budget is the same for every sequence (the reference's batch shares it); a
sub-step over read sets of different sizes runs per sequence.
"""

from __future__ import annotations

import torch

from .fastpath import BlockContext, CompactLayerState, FastLayerPath


class BatchFastPath:
    """caches: one PackedKVCache per sequence (batch_size 1 each, the same heads and
    head_dim); the remaining arguments are FastLayerPath's, shared by every sequence.
    ``paths[i]`` is sequence i's FastLayerPath (its prefix descriptors, step-0 buffers,
    masses and slot masks); its ``states[layer]`` is row i of the layer's shared compact
    buffer."""

    def __init__(self, caches, *, block_size: int, query_indices=(), value_aware: bool = True,
                 sort_indices: bool = True, compute_dtype: torch.dtype = torch.bfloat16, dense_prefix_layers: int = 0,
                 semantic: str = "A"):
        if not caches:
            raise ValueError("a batch needs at least one sequence")
        c0 = caches[0]
        for c in caches:
            if c.batch_size != 1 or c.num_kv_heads != c0.num_kv_heads or c.head_dim != c0.head_dim \
                    or c.device != c0.device:
                raise ValueError("every sequence's cache must hold one sequence of the same heads and head_dim")
        kw = dict(block_size=block_size, query_indices=list(query_indices), value_aware=value_aware,
                  sort_indices=sort_indices, compute_dtype=compute_dtype, dense_prefix_layers=dense_prefix_layers,
                  semantic=semantic)
        self.paths = [FastLayerPath(cache=c, **kw) for c in caches]
        # the batch's own FastLayerPath: its states[layer] is the whole shared compact buffer,
        # so its compact_attention is the batched sub-step (its cache supplies head_dim only)
        self._batch = FastLayerPath(cache=c0, **kw)
        self.block_size = int(block_size)

    @property
    def batch_size(self) -> int:
        return len(self.paths)

    def _ensure_shared(self, layer: int, k: int) -> None:
        """The layer's shared compact buffer with room for k entries and a block, and every
        sequence's state a view of its row."""
        st = self._batch.states.get(layer)
        need = max(1, k) + self.block_size
        if st is not None and st.key.shape[2] >= need:
            return
        c0 = self.paths[0].cache
        shape = (self.batch_size, c0.num_kv_heads, need, c0.head_dim)
        dt = self._batch.compute_dtype
        key = torch.empty(shape, device=c0.device, dtype=dt)
        value = torch.empty(shape, device=c0.device, dtype=dt)
        self._batch.states[layer] = CompactLayerState(key=key, value=value)
        for i, p in enumerate(self.paths):
            p.states[layer] = CompactLayerState(key=key[i:i + 1], value=value[i:i + 1])

    def route(self, layer: int, query: torch.Tensor, current_key: torch.Tensor, current_value: torch.Tensor,
              ctxs) -> torch.Tensor:
        """One layer's attention for the whole batch ([B, Hq, T, D] queries, [B, Hkv, T, D]
        block K/V; ctxs: each sequence's BlockContext, all in the same phase -- step index,
        probe, prefill -- as in one batched forward), routed as FastLayerPath.route routes
        one sequence's: step 0 per sequence into the shared compact buffer, the sub-steps
        of a sparse layer in one batched call.  Returns [B, Hq, T, D]."""
        if query.shape[0] != self.batch_size or len(ctxs) != self.batch_size:
            raise ValueError(f"the batch has {self.batch_size} sequences, got {query.shape[0]} and {len(ctxs)}")
        c0 = ctxs[0]
        phase = lambda c: (c.step_index, c.prefill, c.probe, c.qprobe_start)  # noqa: E731
        if any(phase(c) != phase(c0) for c in ctxs):
            raise ValueError("every sequence of a batched forward is in the same phase (step, probe, prefill)")
        if c0.prefill or c0.probe or c0.qprobe_start is not None or c0.step_index == 0:
            if c0.step_index == 0 and not (c0.prefill or c0.probe or c0.qprobe_start is not None):
                for p, ctx in zip(self.paths, ctxs):
                    if not p.dense_required(layer, ctx):
                        self._ensure_shared(layer, min(ctx.topk, p.prefix(layer).n))
            outs = [p.route(layer, query[i:i + 1], current_key[i:i + 1], current_value[i:i + 1], ctx)
                    for i, (p, ctx) in enumerate(zip(self.paths, ctxs))]
            return torch.cat(outs)
        dense = [p.dense_required(layer, ctx) for p, ctx in zip(self.paths, ctxs)]
        sel = {p.states[layer].selected_k if layer in p.states else 0 for p in self.paths}
        shared = self._batch.states.get(layer)
        if any(dense) or len(sel) != 1 or shared is None or not all(
                p.states.get(layer) is not None and p.states[layer].key.data_ptr() ==
                shared.key[i:i + 1].data_ptr() for i, p in enumerate(self.paths)):
            outs = [p.route(layer, query[i:i + 1], current_key[i:i + 1], current_value[i:i + 1], ctx)
                    for i, (p, ctx) in enumerate(zip(self.paths, ctxs))]
            return torch.cat(outs)
        shared.selected_k = sel.pop()
        return self._batch.compact_attention(layer, query, current_key, current_value)


__all__ = ["BatchFastPath", "BlockContext"]
