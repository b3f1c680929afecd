"""BatchFastPath: a batch of sequences with their own packed caches (ragged prefixes) and
one shared compact buffer per layer, as the reference session's batched CompactLayerState
(session.py:430-454, 1286-1336).  Step 0 equals each sequence's own FastLayerPath bit for
bit (the same per-sequence calls, each read set gathered into its row of the shared
buffer); a sub-step of a sparse layer is one split-K call over the batch, equal to the
per-sequence calls within the attention tolerance (its split boundaries differ) and to the
oracle over each sequence's read set; dense layers, and read sets of different sizes, run
per sequence."""

from __future__ import annotations

import pytest
import torch

from maskahead_amd.cache import PackedKVCache
from maskahead_amd.config import QuantizationConfig
from maskahead_amd.runtime.batch import BatchFastPath
from maskahead_amd.runtime.fastpath import BlockContext, FastLayerPath
from maskahead_amd.workloads import layer_inputs
from oracle import attention as OA

from _util import assert_attention_close

pytestmark = pytest.mark.gpu


def _cache(n, seed, L, gpu, hkv=4, d=128):
    _, k, v, _, _ = layer_inputs(b=1, hq=28, hkv=hkv, d=d, n=n, t=32, seed=seed, dtype=torch.bfloat16)
    c = PackedKVCache(num_layers=L, batch_size=1, num_kv_heads=hkv, head_dim=d, max_tokens=n + 128,
                      quant=QuantizationConfig(residual_tokens=0), device=gpu)
    c.begin_append(n)
    for layer in range(L):
        c.stage_layer(layer, (k + layer).to(gpu), v.to(gpu))
    c.commit_append()
    return c


@pytest.mark.parametrize("lens", [(3000, 4500, 2100), (3000, 400, 2100)])
def test_batch_fast_path_block(gpu, lens):
    L, hq, hkv, d, t, read_k, dense = 3, 28, 4, 128, 32, 512, 1
    B = len(lens)
    caches = [_cache(n, 90 + i, L, gpu) for i, n in enumerate(lens)]
    bp = BatchFastPath(caches, block_size=t, query_indices=list(range(t)), dense_prefix_layers=dense)
    one = [FastLayerPath(cache=c, block_size=t, query_indices=list(range(t)), dense_prefix_layers=dense)
           for c in caches]
    g = torch.Generator().manual_seed(91)
    blocks = [tuple(torch.randn(s, generator=g).to(torch.bfloat16).to(gpu)
                    for s in ((B, hq, t, d), (B, hkv, t, d), (B, hkv, t, d))) for _ in range(L)]
    ctxs = [BlockContext(step_index=0, old_cache_len=n, topk=read_k) for n in lens]
    for layer in range(L):
        q, kc, vc = blocks[layer]
        out = bp.route(layer, q, kc, vc, ctxs)
        want = torch.cat([p.route(layer, q[i:i + 1], kc[i:i + 1], vc[i:i + 1], ctx)
                          for i, (p, ctx) in enumerate(zip(one, ctxs))])
        torch.cuda.synchronize()
        assert torch.equal(out, want), layer
        if layer >= dense:
            for i, p in enumerate(one):
                if p.dense_required(layer, ctxs[i]):           # no read set: a prefix below the budget
                    st = bp.paths[i].states.get(layer)          # (its row of the buffer stays unused)
                    assert layer not in p.states and (st is None or st.selected_k == 0)
                    continue
                k = p.states[layer].selected_k
                assert k == min(read_k, lens[i])
                st = bp.paths[i].states[layer]
                assert st.selected_k == k and torch.equal(st.indices, p.states[layer].indices)
                assert torch.equal(st.key[:, :, :k], p.states[layer].key[:, :, :k])
                assert torch.equal(st.value[:, :, :k], p.states[layer].value[:, :, :k])
    for step in (1, 2):
        for ctx in ctxs:
            ctx.step_index = step
        for layer in range(L):
            q, kc, vc = (x.roll(step, dims=2) for x in blocks[layer])
            out = bp.route(layer, q, kc, vc, ctxs)
            want = torch.cat([p.route(layer, q[i:i + 1], kc[i:i + 1], vc[i:i + 1], ctx)
                              for i, (p, ctx) in enumerate(zip(one, ctxs))])
            torch.cuda.synchronize()
            if layer < dense or min(lens) < read_k:
                assert torch.equal(out, want), (step, layer)      # per-sequence calls
            else:
                assert_attention_close(out, want)
            if layer >= dense:
                for i, p in enumerate(one):
                    if p.dense_required(layer, ctxs[i]):
                        continue
                    st = p.states[layer]
                    k = st.selected_k
                    wo = OA.dense_attention(q[i:i + 1].cpu(), st.key[:, :, :k].cpu(), st.value[:, :, :k].cpu(),
                                            kc[i:i + 1].cpu(), vc[i:i + 1].cpu())
                    assert_attention_close(out[i:i + 1], wo)
    if min(lens) >= read_k:
        # the sparse layers' sub-steps ran as one call over the batch
        assert all(layer in bp._batch._compact_prefix for layer in range(dense, L))
    else:
        assert not bp._batch._compact_prefix


def _snapshot(c):
    names = ("k_q", "k_scale", "k_zero", "v_q", "v_scale", "v_zero", "k_residual", "v_residual")
    cut = {"k_q": c.quantized_length // 32, "k_scale": c.quantized_length // 32, "k_zero": c.quantized_length // 32,
           "v_q": c.quantized_length, "v_scale": c.quantized_length, "v_zero": c.quantized_length,
           "k_residual": c.residual_length, "v_residual": c.residual_length}
    return (c.length, c.quantized_length, c.residual_length), {n: getattr(c, n)[:, :, :, :cut[n]].clone() for n in names}


def test_batch_block_cycle_with_eviction(gpu):
    """Two blocks of a batch as the config-4 bench runs them -- step 0 with per-slot masses,
    lookahead_evict_batch (per_slot), batched sub-steps, the finalize, then a block over the
    rebuilt caches with their dead slots masked -- leave every cache, state, read set and
    step-0 output as the per-sequence path (FastLayerPath with live-order masses and
    lookahead_evict per sequence) does on identical caches; the batched sub-steps agree
    with the per-sequence ones within the attention tolerance."""
    from maskahead_amd.eviction import EvictionConfig, EvictionState
    from maskahead_amd.runtime.session import (admit_new_entries, live_slot_masks, lookahead_evict,
                                               lookahead_evict_batch)

    L, hq, hkv, d, t, read_k, keep_k, W, dense = 3, 28, 4, 128, 32, 256, 1024, 64, 1
    lens = (2400, 3600, 1700)
    B = len(lens)
    cfg = EvictionConfig(policy="lookahead", recent_window=W, capacity_floor=W, compaction="lazy", repack_below=0.5,
                         sink_tokens=4)

    def seqs():
        out = []
        for i, n in enumerate(lens):
            c = _cache(n, 95 + i, L, gpu)
            st = EvictionState(num_layers=L, batch_size=1, num_kv_heads=hkv, capacity=n + 4 * t, device=gpu)
            st.append(range(n))
            out.append((c, st))
        return out

    A, Bq = seqs(), seqs()             # batch path, per-sequence path
    bp = BatchFastPath([c for c, _ in A], block_size=t, query_indices=list(range(t)), dense_prefix_layers=dense)
    one = [FastLayerPath(cache=c, block_size=t, query_indices=list(range(t)), dense_prefix_layers=dense)
           for c, _ in Bq]
    g = torch.Generator().manual_seed(96)
    pos = list(lens)
    for blk in range(2):
        # the slots of the cache as it stands (after the last finalize): dead ones masked
        for (c, st), p in zip(A, bp.paths):
            p.slot_masks = live_slot_masks(c, st)
        for (c, st), p in zip(Bq, one):
            p.slot_masks = live_slot_masks(c, st)
        blocks = [tuple(torch.randn(s, generator=g).to(torch.bfloat16).to(gpu)
                        for s in ((B, hq, t, d), (B, hkv, t, d), (B, hkv, t, d))) for _ in range(L)]
        ctx_a = [BlockContext(step_index=0, old_cache_len=p, topk=read_k, evicting=True, live_len=st.live,
                              want_mass=True) for p, (_, st) in zip(pos, A)]
        ctx_b = [BlockContext(step_index=0, old_cache_len=p, topk=read_k, evicting=True, live_len=st.live,
                              want_mass=True, live_slots={la: st.phys[la, ..., :st.live] for la in range(L)})
                 for p, (_, st) in zip(pos, Bq)]
        for layer in range(L):
            q, kc, vc = blocks[layer]
            out = bp.route(layer, q, kc, vc, ctx_a)
            want = torch.cat([p.route(layer, q[i:i + 1], kc[i:i + 1], vc[i:i + 1], ctx)
                              for i, (p, ctx) in enumerate(zip(one, ctx_b))])
            assert torch.equal(out, want), (blk, layer)
        keeps_a = lookahead_evict_batch([(c, st, p.last_mass, None, n) for (c, st), p, n in zip(A, bp.paths, pos)],
                                        cfg, keep_k, per_slot=True)
        keeps_b = [lookahead_evict(c, st, cfg, keep_k, p.last_mass, None, next_position=n, check=False)
                   for (c, st), p, n in zip(Bq, one, pos)]
        torch.cuda.synchronize()
        for ka, kb, (ca, sa), (cb, sb) in zip(keeps_a, keeps_b, A, Bq):
            assert (ka is None) == (kb is None) and (ka is None or torch.equal(ka, kb))
            sa_, pa = _snapshot(ca)
            sb_, pb = _snapshot(cb)
            assert sa_ == sb_ and all(torch.equal(pa[x], pb[x]) for x in pa)
            assert sa.live == sb.live and torch.equal(sa.phys[..., :sa.live], sb.phys[..., :sb.live])
        for (c, st), p in zip(A, bp.paths):
            p.slot_masks = live_slot_masks(c, st)
        for (c, st), p in zip(Bq, one):
            p.slot_masks = live_slot_masks(c, st)
        for step in (1, 2):
            for ctx in ctx_a + ctx_b:
                ctx.step_index = step
            for layer in range(L):
                q, kc, vc = blocks[layer]
                out = bp.route(layer, q, kc, vc, ctx_a)
                want = torch.cat([p.route(layer, q[i:i + 1], kc[i:i + 1], vc[i:i + 1], ctx)
                                  for i, (p, ctx) in enumerate(zip(one, ctx_b))])
                assert_attention_close(out, want)
        for i, ((ca, sa), (cb, sb)) in enumerate(zip(A, Bq)):
            for c, st in ((ca, sa), (cb, sb)):
                c.begin_append(t)
                for layer in range(L):
                    c.stage_layer(layer, blocks[layer][1][i:i + 1], blocks[layer][2][i:i + 1])
                c.commit_append()
                assert admit_new_entries(c, st, pos[i]) == pos[i] + t
            pos[i] += t
    for (c, _), (c2, _) in zip(A, Bq):
        c.check_rebuild()
        c2.check_rebuild()
