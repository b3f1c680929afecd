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
