"""GPU parity of the cache mirror and the per-layer fast path: PackedKVCache appends
(bf16 and packed int4 with the bf16 residual, cache.py:385-566), views (608-657),
compaction (342-367), and FastLayerPath's step 0 (session.py:1403-1454), sub-step
attention over the compact buffer (1286-1336) and block-causal probe attention with
prefix mass (1378-1392), each against the CPU oracle on the same inputs.  Then BASELINE
config 3's keep/evict step at full size, and config 4's ragged batch at a reduced size."""

import pytest
import torch

from maskahead_amd.cache import PackedKVCache
from maskahead_amd.config import QuantizationConfig
from maskahead_amd.kernels.keep import keep_select, value_score
from maskahead_amd.runtime.fastpath import FastLayerPath
from maskahead_amd.workloads import CONFIGS, layer_inputs
from oracle import attention as OA
from oracle import selection as OS

from _util import assert_attention_close, fastpath_read_set, rel_err

pytestmark = pytest.mark.gpu

BF16 = QuantizationConfig(k_bits=16, v_bits=16)


def _fill(cache, chunks, gpu):
    """Append [B,H,t,D] (K, V) chunk pairs to every layer (layer l gets K + l)."""
    for k, v in chunks:
        cache.begin_append(k.shape[2])
        for l in range(cache.num_layers):
            cache.stage_layer(l, (k + l).to(torch.bfloat16).to(gpu), v.to(torch.bfloat16).to(gpu))
        cache.commit_append()


def _oracle_packed_layer(k, v, residual_tokens=32, kg=32):
    """What a packed cache holds after one append of [B,H,n,D] bf16 K/V: the first `move`
    tokens quantized (oracle rule, bf16 arithmetic) and dequantized, the rest bf16."""
    n = k.shape[2]
    move = (max(0, n - residual_tokens) // kg) * kg
    kb, vb = k.to(torch.bfloat16), v.to(torch.bfloat16)
    kd = OA.dequantize_keys(*OA.quantize_keys(kb[:, :, :move])).to(torch.bfloat16)
    vd = OA.dequantize_values(*OA.quantize_values(vb[:, :, :move])).to(torch.bfloat16)
    return torch.cat([kd, kb[:, :, move:]], 2), torch.cat([vd, vb[:, :, move:]], 2), move


def test_cache_bf16_append_view_compact(gpu):
    g = torch.Generator().manual_seed(21)
    L, B, H, D = 2, 1, 4, 128
    c = PackedKVCache(num_layers=L, batch_size=B, num_kv_heads=H, head_dim=D, max_tokens=8192, quant=BF16,
                      device=gpu)
    k1, v1 = torch.randn((B, H, 3000, D), generator=g), torch.randn((B, H, 3000, D), generator=g)
    k2, v2 = torch.randn((B, H, 32, D), generator=g), torch.randn((B, H, 32, D), generator=g)
    _fill(c, [(k1, v1), (k2, v2)], gpu)
    assert c.length == 3032 and c.get_seq_length() == 3032 and c.capacity >= 3032
    kall, vall = torch.cat([k1, k2], 2), torch.cat([v1, v2], 2)
    for l in range(L):
        view = c.layer_view(l)
        assert view.length == 3032 and view.k_fp.shape[2] == 3032
        assert torch.equal(view.k_fp.cpu(), (kall + l).to(torch.bfloat16))
        assert torch.equal(view.v_fp.cpu(), vall.to(torch.bfloat16))
    pos = torch.arange(3032).expand(L, B, H, 3032)
    score = torch.rand((L, B, H, 3032), generator=g)
    keep = OS.keep_select(pos.reshape(-1, 3032), score.reshape(-1, 3032), 700, 64, 4).view(L, B, H, 700)
    before = [(c.layer_view(l).k_fp.cpu().clone(), c.layer_view(l).v_fp.cpu().clone()) for l in range(L)]
    c.compact(keep.to(gpu))
    assert c.length == 700 and c.dropped == 2332 and c.get_seq_length() == 3032
    for l in range(L):
        gi = keep[l].unsqueeze(-1).expand(-1, -1, -1, D)
        assert torch.equal(c.layer_view(l).k_fp.cpu(), before[l][0].gather(2, gi))
        assert torch.equal(c.layer_view(l).v_fp.cpu(), before[l][1].gather(2, gi))
    # the next block lands right after the survivors
    _fill(c, [(k2 * 2, v2 * 2)], gpu)
    assert c.length == 732
    assert torch.equal(c.layer_view(1).k_fp[:, :, 700:].cpu(), (k2 * 2 + 1).to(torch.bfloat16))


def test_cache_packed_append_residual_and_compact(gpu):
    g = torch.Generator().manual_seed(22)
    L, B, H, D = 2, 1, 4, 128
    q4 = QuantizationConfig()           # k4v4, groups of 32, 32 residual tokens
    c = PackedKVCache(num_layers=L, batch_size=B, num_kv_heads=H, head_dim=D, max_tokens=8192, quant=q4,
                      device=gpu)
    k1 = torch.randn((B, H, 1000, D), generator=g) * torch.empty((1, H, 1, D)).log_normal_(0, 0.5, generator=g)
    v1 = torch.randn((B, H, 1000, D), generator=g)
    _fill(c, [(k1, v1)], gpu)
    assert (c.length, c.quantized_length, c.residual_length) == (1000, 960, 40)
    for l in range(L):
        wk, wv, move = _oracle_packed_layer(k1 + l, v1)
        gk, gv = c.dequantize_layer(l)
        assert torch.equal(gk.cpu(), wk) and torch.equal(gv.cpu(), wv)
    # a block of 32: the residual (40) + 32 -> one more key group is quantized
    k2, v2 = torch.randn((B, H, 32, D), generator=g), torch.randn((B, H, 32, D), generator=g)
    _fill(c, [(k2, v2)], gpu)
    assert (c.length, c.quantized_length, c.residual_length) == (1032, 992, 40)
    kall, vall = torch.cat([k1, k2], 2), torch.cat([v1, v2], 2)
    wk, wv, _ = _oracle_packed_layer(kall, vall)
    gk, gv = c.dequantize_layer(0)
    assert torch.equal(gk.cpu(), wk) and torch.equal(gv.cpu(), wv)
    # compaction of a packed cache: survivors gathered dequantized, then re-appended
    keep = torch.sort(torch.randperm(1032, generator=g)[:500]).values.expand(L, B, H, 500).contiguous()
    before = [c.dequantize_layer(l) for l in range(L)]
    c.compact(keep.to(gpu))
    assert c.length == 500 and c.dropped == 532
    for l in range(L):
        gi = keep[l].unsqueeze(-1).expand(-1, -1, -1, D)
        sk, sv = before[l][0].cpu().gather(2, gi), before[l][1].cpu().gather(2, gi)
        wk, wv, _ = _oracle_packed_layer(sk, sv)
        gk, gv = c.dequantize_layer(l)
        assert torch.equal(gk.cpu(), wk) and torch.equal(gv.cpu(), wv)


@pytest.mark.parametrize("packed,t", [(False, 32), (True, 32), (True, 8)])
def test_fastpath_step0_substeps_probe(gpu, packed, t):
    hq, hkv, d, n, k_read = 28, 4, 128, 4096, 512
    q, k, v, kc, vc = layer_inputs(b=1, hq=hq, hkv=hkv, d=d, n=n, t=t, seed=31)
    quant = QuantizationConfig() if packed else BF16
    cache = PackedKVCache(num_layers=1, batch_size=1, num_kv_heads=hkv, head_dim=d, max_tokens=8192, quant=quant,
                          device=gpu)
    _fill(cache, [(k, v)], gpu)
    if packed:
        kd, vd, _ = _oracle_packed_layer(k, v)
    else:
        kd, vd = k.to(torch.bfloat16), v.to(torch.bfloat16)
    fp = FastLayerPath(cache=cache, block_size=t, query_indices=list(range(t)))
    qb, kcb, vcb = q.to(torch.bfloat16), kc.to(torch.bfloat16), vc.to(torch.bfloat16)
    qg, kcg, vcg = qb.to(gpu), kcb.to(gpu), vcb.to(gpu)

    # step 0: attention over [prefix | block], value-aware read set, gather
    out = fp.step0(0, qg, kcg, vcg, select=True, topk=k_read)
    wout, wmp, wlp, wop = OA.splitk_attention(qb, kd, vd, kcb, vcb)
    assert_attention_close(out, wout)
    fastpath_read_set(f"fastpath_step0_{'k4v4' if packed else 'bf16'}_t{t}", fp, 0, qg, kcg, vcg, kd, vd,
                      range(t), k_read, (wmp, wlp, wop))
    st = fp.states[0]
    idx = st.indices.cpu()
    gi = idx.unsqueeze(-1).expand(-1, -1, -1, d)
    assert torch.equal(st.key[:, :, :k_read].cpu(), kd.gather(2, gi))
    assert torch.equal(st.value[:, :, :k_read].cpu(), vd.gather(2, gi))

    # sub-steps: attention over [selected | new block K/V]
    g = torch.Generator().manual_seed(32)
    for _ in range(2):
        q2 = torch.randn((1, hq, t, d), generator=g).to(torch.bfloat16)
        k2 = torch.randn((1, hkv, t, d), generator=g).to(torch.bfloat16)
        v2 = torch.randn((1, hkv, t, d), generator=g).to(torch.bfloat16)
        got = fp.compact_attention(0, q2.to(gpu), k2.to(gpu), v2.to(gpu))
        want = OA.dense_attention(q2, kd.gather(2, gi), vd.gather(2, gi), k2, v2)
        assert got.dtype == torch.bfloat16
        assert_attention_close(got, want)

    # probe: block-causal attention (blocks of 8) with the prefix mass of chosen rows
    rows = [0, 3, t - 1]
    out_p, mass = fp.attend(0, qg, kcg, vcg, causal=8, q_pos0=n, mass_rows=rows)
    wout_p, wmp_p, wlp_p, _ = OA.splitk_attention(qb, kd, vd, kcb, vcb, causal_block=8, q_pos0=n, c_pos0=n)
    assert_attention_close(out_p, wout_p)
    wmass, _ = OA.prefix_scores(qb, kd, None, wmp_p, wlp_p, None, rows, value_aware=False)
    assert rel_err(mass, wmass) < 1e-4


def test_config3_keep_step(gpu):
    """BASELINE config 3 at full size: bf16 prefix 65536, 32/8 heads, 96 probe rows (the
    block + 2 look-ahead blocks, block-causal), keep 8192 per KV head, then the
    finalized block appended after the survivors."""
    sh = CONFIGS["c3"]
    q, k, v, kc, vc = layer_inputs(sh, dtype=torch.bfloat16)
    cache = PackedKVCache(num_layers=1, batch_size=1, num_kv_heads=sh.hkv, head_dim=sh.d, max_tokens=sh.n + 64,
                          quant=BF16, device=gpu)
    _fill(cache, [(k, v)], gpu)
    fp = FastLayerPath(cache=cache, block_size=32, query_indices=list(range(32)))
    qg, kcg, vcg = q.to(gpu), kc.to(gpu), vc.to(gpu)
    out, mass = fp.attend(0, qg, kcg, vcg, causal=32, q_pos0=sh.n, mass_rows=list(range(sh.t)))
    # oracle on two KV heads (8 query heads): enough rows to pin the kernels, CPU-cheap
    hs = slice(0, 2)
    wout, wmp, wlp, _ = OA.splitk_attention(q[:, :8], k[:, hs], v[:, hs], kc[:, hs], vc[:, hs], causal_block=32,
                                            q_pos0=sh.n, c_pos0=sh.n)
    assert_attention_close(out[:, :8], wout)
    wmass, _ = OA.prefix_scores(q[:, :8], k[:, hs], None, wmp, wlp, None, range(sh.t), value_aware=False)
    assert rel_err(mass[:, hs], wmass) < 1e-4
    assert torch.all(mass >= 0)
    # keep score and keep set on the GPU's own mass: bit-exact against the oracle
    view = cache.layer_view(0)
    score = value_score(mass, view.v_fp)
    wscore = OA.value_score_bf16(mass.cpu(), v)
    assert torch.equal(score.cpu(), wscore)
    pos = torch.arange(sh.n, dtype=torch.int32).expand(1, 1, sh.hkv, sh.n)
    keep = keep_select(pos.to(gpu), score.unsqueeze(0), sh.keep_k, 128, sink_tokens=4)
    wkeep = OS.keep_select(pos.reshape(-1, sh.n), wscore.reshape(-1, sh.n), sh.keep_k, 128, 4)
    assert torch.equal(keep.cpu().reshape(-1, sh.keep_k), wkeep)
    # compaction in place, then the finalized block appended after the survivors
    cache.compact(keep)
    assert cache.length == sh.keep_k and cache.get_seq_length() == sh.n
    gi = wkeep.view(1, sh.hkv, sh.keep_k, 1).expand(-1, -1, -1, sh.d)
    assert torch.equal(cache.layer_view(0).k_fp.cpu(), k.gather(2, gi))
    assert torch.equal(cache.layer_view(0).v_fp.cpu(), v.gather(2, gi))
    _fill(cache, [(kc[:, :, :32], vc[:, :, :32])], gpu)
    assert cache.length == sh.keep_k + 32
    assert torch.equal(cache.layer_view(0).k_fp[:, :, sh.keep_k:].cpu(), kc[:, :, :32])


def test_config4_ragged_batch_step0_and_keep(gpu):
    """BASELINE config 4's structure at a CPU-checkable size: a batch of sequences with
    different prefix lengths in one packed int4 cache (the slots past each sequence's
    length dead in the layer's slot mask), two layers of the config-1 head shape, step 0
    of every layer (attention, value-aware read set of 512 over live slots, gather), then
    each sequence's keep set (budget 1024, window 64, 4 sinks) over its live entries."""
    b, hq, hkv, d, t, k_read, keep_k = 3, 28, 4, 128, 32, 512, 1024
    lens = [1536, 3200, 4064]
    n = max(lens)
    q, k, v, kc, vc = layer_inputs(b=b, hq=hq, hkv=hkv, d=d, n=n, t=t, seed=44)
    cache = PackedKVCache(num_layers=2, batch_size=b, num_kv_heads=hkv, head_dim=d, max_tokens=n + 64,
                          quant=QuantizationConfig(), device=gpu)
    _fill(cache, [(k, v)], gpu)
    mask = torch.zeros((b, hkv, n), dtype=torch.uint8)
    for i, ln in enumerate(lens):
        mask[i, :, :ln] = 1
    fp = FastLayerPath(cache=cache, block_size=t, query_indices=list(range(t)),
                       slot_masks={l: mask.to(gpu) for l in range(2)})
    qb, kcb, vcb = q.to(torch.bfloat16), kc.to(torch.bfloat16), vc.to(torch.bfloat16)
    for layer in range(2):
        kd, vd, _ = _oracle_packed_layer(k + layer, v)
        out = fp.step0(layer, qb.to(gpu), kcb.to(gpu), vcb.to(gpu), select=True, topk=k_read, want_mass=True)
        wout, wmp, wlp, wop = OA.splitk_attention(qb, kd, vd, kcb, vcb, mask=mask)
        assert_attention_close(out, wout)
        wmass, _ = OA.prefix_scores(qb, kd, vd.float(), wmp, wlp, wop, list(range(t)), mask=mask,
                                    value_aware=True)
        assert rel_err(fp.last_mass[layer].cpu() + (1 - mask), wmass + (1 - mask)) < 1e-4
        fastpath_read_set(f"ragged_batch_layer{layer}", fp, layer, qb.to(gpu), kcb.to(gpu), vcb.to(gpu), kd, vd,
                          range(t), k_read, (wmp, wlp, wop), mask=mask)
        st = fp.states[layer]
        idx = st.indices.cpu()
        assert bool(torch.all(mask.gather(2, idx) == 1))          # only live slots are read
        gi = idx.unsqueeze(-1).expand(-1, -1, -1, d)
        assert torch.equal(st.key[:, :, :k_read].cpu(), kd.gather(2, gi))
        assert torch.equal(st.value[:, :, :k_read].cpu(), vd.gather(2, gi))
        # eviction: each sequence's keep set over its live entries, bit-exact vs the oracle
        mass = fp.last_mass[layer]
        for i, ln in enumerate(lens):
            pos = torch.arange(ln, dtype=torch.int64).expand(1, hkv, ln)
            sc = mass[i:i + 1, :, :ln]
            keep = keep_select(pos.to(gpu), sc, keep_k, 64, sink_tokens=4)
            wkeep = OS.keep_select(pos.reshape(-1, ln), sc.cpu().reshape(-1, ln), keep_k, 64, 4)
            assert torch.equal(keep.cpu().reshape(-1, keep_k), wkeep), (layer, i)
