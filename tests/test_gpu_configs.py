"""GPU parity at the benchmark configurations' own sizes (BASELINE configs 1 and 4).

* Config 1: one bf16 layer, prefix 32 768, 28/4 heads, block 32, read 2 048: step 0
  (attention, value-aware scores, read set, gather) and 3 denoising sub-steps over the
  compact buffer (session.py:1403-1454, 1286-1336), all against the oracle.
* Config 4: 8 sequences with prefix lengths drawn uniform in [8 192, 131 072] (seed 1234),
  28 layers (2 dense + 26 sparse), packed int4, read 2 048 / keep 4 096 per KV head: for
  each sequence one block -- step 0 of every layer, the lookahead eviction that follows it
  (keep set + packed lazy rebuild, session.py:1985-2034, 270-361), 3 sub-steps, and the
  block's finalize (its KV appended).  The oracle checks the shortest and the longest
  sequence on one dense and one sparse layer (all KV heads), every keep set (bit-exact) and
  the rebuilt cache of the shortest sequence (bit-exact); every sparse layer of every
  sequence, all KV heads, has its read set equal to the oracle's top-k of the scores the
  same passes give (bit-exact) and its step-0 mass equal to theirs; every other layer and
  sequence gets the invariants (finite outputs; read sets ascending, unique, live, of the
  budget)."""

from __future__ import annotations

import pytest
import torch

from maskahead_amd.cache import PackedKVCache
from maskahead_amd.config import QuantizationConfig
from maskahead_amd.eviction import EvictionConfig, EvictionState
from maskahead_amd.kernels.splitk import prefix_scores, splitk_attention
from maskahead_amd.runtime.fastpath import BlockContext, FastLayerPath
from maskahead_amd.runtime.session import admit_new_entries, live_slot_masks, lookahead_evict, lookahead_scores
from maskahead_amd.workloads import CONFIGS, layer_inputs
from oracle import attention as OA
from oracle import rebuild as OR
from oracle import selection as OS

from _util import assert_attention_close, check_read_set, same_bits

pytestmark = pytest.mark.gpu

BF16 = QuantizationConfig(k_bits=16, v_bits=16)
STORE = (("kq", "k_q"), ("ks", "k_scale"), ("kz", "k_zero"), ("vq", "v_q"), ("vs", "v_scale"), ("vz", "v_zero"),
         ("kr", "k_residual"), ("vr", "v_residual"))


def test_config1_block_step_full_size(gpu):
    sh = CONFIGS["c1"]
    q, k, v, kc, vc = layer_inputs(sh, dtype=torch.bfloat16)
    cache = PackedKVCache(num_layers=1, batch_size=1, num_kv_heads=sh.hkv, head_dim=sh.d, max_tokens=sh.n + 64,
                          quant=BF16, device=gpu)
    cache.begin_append(sh.n)
    cache.stage_layer(0, k.to(gpu), v.to(gpu))
    cache.commit_append()
    fp = FastLayerPath(cache=cache, block_size=sh.t, query_indices=list(range(sh.t)))
    qg, kcg, vcg = q.to(gpu), kc.to(gpu), vc.to(gpu)
    out = fp.step0(0, qg, kcg, vcg, select=True, topk=sh.read_k)
    wout, wmp, wlp, wop = OA.splitk_attention(q, k, v, kc, vc)
    assert_attention_close(out, wout)
    # the scores step 0 ranked (the same deterministic passes), and the oracle's from the
    # GPU's statistics and from its own
    pre = fp.prefix(0)
    _, st = splitk_attention(qg, pre, kcg, vcg, want_prefix=True)
    _, gscore = prefix_scores(qg, pre, st, torch.arange(sh.t, dtype=torch.int32), value=True)
    gmp, glp, gop = (x.cpu() for x in st[:3])
    rows = list(range(sh.t))
    _, sscore = OA.prefix_scores(q, k, v.float(), gmp, glp, gop, rows, value_aware=True)
    _, wscore = OA.prefix_scores(q, k, v.float(), wmp, wlp, wop, rows, value_aware=True)
    idx = fp.states[0].indices.cpu()
    check_read_set("c1_step0", idx, gscore.cpu(), sscore, wscore, sh.read_k)
    assert torch.all(idx[..., 1:] > idx[..., :-1])
    gi = idx.unsqueeze(-1).expand(-1, -1, -1, sh.d)
    ks, vs = k.gather(2, gi), v.gather(2, gi)
    assert torch.equal(fp.states[0].key[:, :, :sh.read_k].cpu(), ks)
    assert torch.equal(fp.states[0].value[:, :, :sh.read_k].cpu(), vs)
    g = torch.Generator().manual_seed(4321)
    for _ in range(3):
        q2 = torch.randn((1, sh.hq, sh.t, sh.d), generator=g).to(torch.bfloat16)
        k2 = torch.randn((1, sh.hkv, sh.t, sh.d), generator=g).to(torch.bfloat16)
        v2 = torch.randn((1, sh.hkv, sh.t, sh.d), generator=g).to(torch.bfloat16)
        got = fp.compact_attention(0, q2.to(gpu), k2.to(gpu), v2.to(gpu))
        assert_attention_close(got, OA.dense_attention(q2, ks, vs, k2, v2))


def _seq_inputs(n: int, seed: int, gpu, layers: int, hkv=4, hq=28, d=128, t=32):
    """Per-sequence seeded K/V (the benchmark distribution, drawn on the GPU: N(0,1) with
    LogNormal(0, 0.5) key channels and 4 sink keys x8) and per-layer block tensors."""
    g = torch.Generator(device=gpu).manual_seed(seed)
    chan = torch.empty((1, hkv, 1, d), device=gpu).log_normal_(0.0, 0.5, generator=g)
    k = torch.randn((1, hkv, n, d), device=gpu, generator=g) * chan
    k[:, :, :4] *= 8.0
    v = torch.randn((1, hkv, n, d), device=gpu, generator=g)
    blocks = []
    for _ in range(layers):
        blocks.append(tuple(x.to(torch.bfloat16) for x in (
            torch.randn((1, hq, t, d), device=gpu, generator=g), torch.randn((1, hkv, t, d), device=gpu, generator=g)
            * chan, torch.randn((1, hkv, t, d), device=gpu, generator=g))))
    return k.to(torch.bfloat16), v.to(torch.bfloat16), blocks


def _oracle_view(cache, layer):
    """The oracle's K/V of one stored layer: packed part dequantized on the CPU from the raw
    bytes (reference.py:168-179, 259-268), then the bf16 residual."""
    view = cache.layer_view(layer)
    parts_k, parts_v = [], []
    if view.quantized_length:
        parts_k.append(OA.dequantize_keys(view.k_q.cpu(), view.k_scale.cpu(), view.k_zero.cpu()).to(torch.bfloat16))
        parts_v.append(OA.dequantize_values(view.v_q.cpu(), view.v_scale.cpu(), view.v_zero.cpu()).to(torch.bfloat16))
    if view.residual_length:
        parts_k.append(view.k_residual.cpu())
        parts_v.append(view.v_residual.cpu())
    return torch.cat(parts_k, 2), torch.cat(parts_v, 2)


def _check_read_set_invariants(idx, n, k, mask=None):
    ic = idx.cpu()
    assert ic.shape[-1] == k
    assert torch.all(ic[..., 1:] > ic[..., :-1]) and int(ic.min()) >= 0 and int(ic.max()) < n
    if mask is not None:
        assert bool(torch.all(mask.cpu().gather(-1, ic) == 1))


def test_config4_ragged_block_step(gpu):
    L, hq, hkv, d, t, read_k, keep_k, W, dense = 28, 28, 4, 128, 32, 2048, 4096, 64, 2
    lens = torch.randint(8192, 131073, (8,), generator=torch.Generator().manual_seed(1234)).tolist()
    smallest, largest = lens.index(min(lens)), lens.index(max(lens))
    quant = QuantizationConfig(residual_tokens=0)          # ours_k4v4: every whole group quantized
    cfg = EvictionConfig(policy="lookahead", recent_window=W, capacity_floor=512, compaction="lazy",
                         repack_below=1.0, sink_tokens=4)
    for i, n in enumerate(lens):
        k, v, blocks = _seq_inputs(n, 1234 + i, gpu, L)
        cache = PackedKVCache(num_layers=L, batch_size=1, num_kv_heads=hkv, head_dim=d, max_tokens=n + 4 * t,
                              quant=quant, device=gpu)
        cache.begin_append(n)
        for layer in range(L):
            cache.stage_layer(layer, torch.roll(k, 977 * layer, dims=2), v)
        cache.commit_append()
        del k, v
        st = EvictionState(num_layers=L, batch_size=1, num_kv_heads=hkv, capacity=n + 4 * t, device=gpu)
        st.append(range(n))
        fp = FastLayerPath(cache=cache, block_size=t, query_indices=list(range(t)), dense_prefix_layers=dense)
        check = i in (smallest, largest)
        checked = (0, L - 1) if check else ()
        views = {layer: _oracle_view(cache, layer) for layer in checked}
        pre_store = ({s: getattr(cache, a).cpu() for s, a in STORE},
                     (cache.length, cache.quantized_length, cache.residual_length, cache.dropped)) \
            if i == smallest else None
        ctx = BlockContext(step_index=0, old_cache_len=n, topk=read_k, evicting=True, live_len=st.live,
                           want_mass=True, live_slots={layer: st.phys[layer, ..., :st.live] for layer in range(L)})
        # step 0 of every layer
        for layer in range(L):
            q, kc, vc = blocks[layer]
            out = fp.route(layer, q, kc, vc, ctx)
            assert torch.isfinite(out.float()).all()
            if layer >= dense:
                _check_read_set_invariants(fp.states[layer].indices, n, read_k)
                # every sparse layer, every KV head: the read set is the oracle's top-k of
                # the scores the same passes give, and step 0 kept their mass
                pre = fp.prefix(layer)
                _, sts = splitk_attention(q, pre, kc, vc, want_prefix=True)
                gmass, gscore = prefix_scores(q, pre, sts, torch.arange(t, dtype=torch.int32), value=True)
                assert torch.equal(fp.last_mass[layer], gmass)
                assert torch.equal(fp.states[layer].indices.cpu(), OS.topk_ascending(gscore.cpu(), read_k)), \
                    (i, layer)
            else:
                assert layer not in fp.states
            if layer in checked:
                kd, vd = views[layer]
                qc, kcc, vcc = q.cpu(), kc.cpu(), vc.cpu()
                wout, wmp, wlp, wop = OA.splitk_attention(qc, kd, vd, kcc, vcc)
                assert_attention_close(out, wout)
                if layer >= dense:
                    gmp, glp, gop = (x.cpu() for x in sts[:3])
                    rows = list(range(t))
                    _, sscore = OA.prefix_scores(qc, kd, vd.float(), gmp, glp, gop, rows,
                                                 value_aware=True)
                    _, wscore = OA.prefix_scores(qc, kd, vd.float(), wmp, wlp, wop, rows,
                                                 value_aware=True)
                    check_read_set(f"c4_seq{i}_n{n}_layer{layer}", fp.states[layer].indices.cpu(), gscore.cpu(), sscore,
                                   wscore, read_k)
        # the lookahead eviction after step 0 (finish_step0): keep set on the GPU's scores
        pos0 = st.pos[..., :st.live].cpu().to(torch.int64)
        phys0 = st.phys[..., :st.live].cpu().to(torch.int64)
        score = lookahead_scores(cache, st, fp.last_mass, None, use_value=True)
        keep = lookahead_evict(cache, st, cfg, keep_k, fp.last_mass, None, next_position=n)
        torch.cuda.synchronize()
        assert keep is not None and st.live == keep_k
        want_keep = OS.keep_select(pos0.reshape(-1, n), score.cpu().reshape(-1, n), keep_k, W, 4)
        assert torch.equal(keep.cpu().reshape(-1, keep_k), want_keep), i
        if pre_store is not None:
            new, new_lens, new_phys = OR.evict(pre_store[0], pre_store[1], pos0, phys0, keep.cpu(), next_position=n,
                                               stage_mode=False, mode="lazy", repack_below=1.0, recent_window=W)
            assert (cache.length, cache.quantized_length, cache.residual_length, cache.dropped) == new_lens
            assert torch.equal(st.phys[..., :keep_k].cpu().to(torch.int64), new_phys)
            ng, ql, rl = new_lens[1] // 32, new_lens[1], new_lens[2]
            for short, name in STORE:
                cut = ng if short in ("kq", "ks", "kz") else ql if short in ("vq", "vs", "vz") else rl
                assert same_bits(getattr(cache, name)[:, :, :, :cut], new[short]), short
        # 3 sub-steps: sparse layers over their read sets, dense layers over the survivors
        fp.slot_masks = live_slot_masks(cache, st)
        for step in (1, 2, 3):
            ctx.step_index = step
            for layer in range(L):
                q, kc, vc = blocks[layer]
                out = fp.route(layer, q, kc, vc, ctx)
                assert torch.isfinite(out.float()).all()
                if step == 1 and layer == L - 1 and check:
                    kd, vd = views[layer]
                    gi = fp.states[layer].indices.cpu().unsqueeze(-1).expand(-1, -1, -1, d)
                    want = OA.dense_attention(q.cpu(), kd.gather(2, gi), vd.gather(2, gi), kc.cpu(), vc.cpu())
                    assert_attention_close(out, want)
        # the block's finalize: its KV appended, its positions admitted
        cache.begin_append(t)
        for layer in range(L):
            cache.stage_layer(layer, blocks[layer][1], blocks[layer][2])
        cache.commit_append()
        assert admit_new_entries(cache, st, n) == n + t
        assert st.live == keep_k + t and cache.get_seq_length() == n + t
        # the admitted entries hold the newest physical slots (the cache was compacted)
        assert torch.equal(st.phys[..., keep_k:keep_k + t].cpu(),
                           torch.arange(cache.length - t, cache.length, dtype=torch.int32).expand(L, 1, hkv, t))
        del cache, st, fp, blocks
        torch.cuda.empty_cache()
