"""The lookahead eviction lifecycle on a packed cache (session.py:1985-2034, 2317-2332,
270-361, 240-255), stage by stage against the oracle: step-0 prefix mass, a block-causal
probe of the next blocks, the lookahead score value_score(a1 + a_probe, v_live), the keep
set, the lazy rebuild, and attention over the rebuilt cache with its dead slots masked."""

from __future__ import annotations

import pytest
import torch

from maskahead_amd.cache import PackedKVCache
from maskahead_amd.config import QuantizationConfig
from maskahead_amd.eviction import EvictionConfig, EvictionState
from maskahead_amd.runtime.fastpath import FastLayerPath
from maskahead_amd.runtime.session import live_slot_masks, lookahead_evict, lookahead_scores
from maskahead_amd.workloads import layer_inputs
from oracle import attention as OA
from oracle import rebuild as OR
from oracle import selection as OS
from tests._util import assert_attention_close, rel_err, same_bits

pytestmark = pytest.mark.gpu

STORE = (("kq", "k_q"), ("ks", "k_scale"), ("kz", "k_zero"), ("vq", "v_q"), ("vs", "v_scale"), ("vz", "v_zero"),
         ("kr", "k_residual"), ("vr", "v_residual"))


def _snapshot(cache):
    lens = (cache.length, cache.quantized_length, cache.residual_length, cache.dropped)
    return {short: getattr(cache, name).cpu() for short, name in STORE}, lens


def test_lookahead_probe_evict_then_masked_attention(gpu):
    L, hq, hkv, d, n, t, C, W = 2, 28, 4, 128, 4096, 32, 1024, 64
    q, k, v, kc, vc = layer_inputs(b=1, hq=hq, hkv=hkv, d=d, n=n, t=t, seed=41)
    cache = PackedKVCache(num_layers=L, batch_size=1, num_kv_heads=hkv, head_dim=d, max_tokens=1 << 16,
                          quant=QuantizationConfig(), device=gpu)
    cache.begin_append(n)
    for layer in range(L):
        cache.stage_layer(layer, (k + layer).to(torch.bfloat16).to(gpu), v.to(torch.bfloat16).to(gpu))
    cache.commit_append()
    st = EvictionState(num_layers=L, batch_size=1, num_kv_heads=hkv, capacity=n, device=gpu)
    st.append(range(n))
    fp = FastLayerPath(cache=cache, block_size=t, query_indices=list(range(t)))
    qb, kcb, vcb = q.to(torch.bfloat16), kc.to(torch.bfloat16), vc.to(torch.bfloat16)
    g = torch.Generator().manual_seed(42)
    qp = torch.randn((1, hq, 3 * t, d), generator=g).to(torch.bfloat16)
    kp = torch.randn((1, hkv, 3 * t, d), generator=g).to(torch.bfloat16)
    vp = torch.randn((1, hkv, 3 * t, d), generator=g).to(torch.bfloat16)
    store0, lens0 = _snapshot(cache)
    deq = OR._dequantize_all(store0, lens0)            # the oracle's view of every layer, bf16

    a1 = {}
    for layer in range(L):
        kd, vd = deq[0][layer], deq[1][layer]
        # step 0 of the block: attention and the prefix mass of its queries
        fp.step0(layer, qb.to(gpu), kcb.to(gpu), vcb.to(gpu), select=False, topk=1, want_mass=True)
        a1[layer] = fp.last_mass[layer]
        _, mp, lp, _ = OA.splitk_attention(qb, kd, vd, kcb, vcb)
        wmass, _ = OA.prefix_scores(qb, kd, None, mp, lp, None, list(range(t)), value_aware=False)
        assert rel_err(a1[layer], wmass) < 1e-4
        # probe of blocks k+1 .. k+3: block-causal, the mass of blocks k+2, k+3 counted per block
        out_p = fp.probe(layer, qp.to(gpu), kp.to(gpu), vp.to(gpu), live_slots=st.phys[layer, ..., :st.live])
        wout_p, mpp, lpp, _ = OA.splitk_attention(qp, kd, vd, kp, vp, causal_block=t, q_pos0=0, c_pos0=0)
        assert_attention_close(out_p, wout_p)
        wpm, _ = OA.prefix_scores(qp, kd, None, mpp, lpp, None, list(range(t, 3 * t)), value_aware=False)
        assert rel_err(fp.probe_mass[layer], wpm * 2) < 1e-4

    # the lookahead score from the GPU masses: value_score in bf16, bit-exact
    score = lookahead_scores(cache, st, a1, fp.probe_mass, use_value=True)
    for layer in range(L):
        a = (a1[layer] + fp.probe_mass[layer]).cpu()
        want = OA.value_score_bf16(a, deq[1][layer])
        assert torch.equal(score[layer].cpu(), want)

    cfg = EvictionConfig(policy="lookahead", recent_window=W, capacity_floor=W, compaction="lazy",
                         repack_below=0.25)
    pos0, phys0 = st.pos[..., :n].cpu().to(torch.int64), st.phys[..., :n].cpu().to(torch.int64)
    keep = lookahead_evict(cache, st, cfg, C, a1, fp.probe_mass, next_position=n)
    torch.cuda.synchronize()
    want_keep = OS.keep_select(pos0, score.cpu(), C, W)
    assert torch.equal(keep.cpu(), want_keep)
    new, new_lens, new_phys = OR.evict(store0, lens0, pos0, phys0, want_keep, next_position=n, stage_mode=False,
                                       mode="lazy", repack_below=0.25, recent_window=W)
    assert (cache.length, cache.quantized_length, cache.residual_length, cache.dropped) == new_lens
    assert torch.equal(st.phys[..., :C].cpu().to(torch.int64), new_phys)
    ng, ql, rl = new_lens[1] // 32, new_lens[1], new_lens[2]
    for short, name in STORE:
        cut = ng if short in ("kq", "ks", "kz") else ql if short in ("vq", "vs", "vz") else rl
        assert same_bits(getattr(cache, name)[:, :, :, :cut], new[short]), short
    assert cache.length > C          # kept groups carry dead slots: the masks matter

    # attention of the next block over the rebuilt cache, dead slots masked
    fp.slot_masks = live_slot_masks(cache, st)
    q3 = torch.randn((1, hq, t, d), generator=g).to(torch.bfloat16)
    k3 = torch.randn((1, hkv, t, d), generator=g).to(torch.bfloat16)
    v3 = torch.randn((1, hkv, t, d), generator=g).to(torch.bfloat16)
    kd2, vd2 = OR._dequantize_all(new, new_lens)
    for layer in range(L):
        out, _ = fp.attend(layer, q3.to(gpu), k3.to(gpu), v3.to(gpu))
        gi = new_phys[layer].unsqueeze(-1).expand(-1, -1, -1, d)
        want = OA.dense_attention(q3, kd2[layer].gather(2, gi), vd2[layer].gather(2, gi), k3, v3)
        assert_attention_close(out, want)

    # a second cycle over the rebuilt cache, where the slots of the live entries are no
    # longer 0..live-1: step 0 and the probe hand back their masses in live order, the
    # lookahead score and the keep set follow from them
    live = st.live
    assert not torch.equal(new_phys[0], torch.arange(live).expand_as(new_phys[0]))
    a1b = {}
    qp2 = torch.randn((1, hq, 2 * t, d), generator=g).to(torch.bfloat16)
    kp2 = torch.randn((1, hkv, 2 * t, d), generator=g).to(torch.bfloat16)
    vp2 = torch.randn((1, hkv, 2 * t, d), generator=g).to(torch.bfloat16)
    for layer in range(L):
        slots = st.phys[layer, ..., :live]
        mask = fp.slot_masks[layer].cpu()
        fp.step0(layer, q3.to(gpu), k3.to(gpu), v3.to(gpu), select=False, topk=1, want_mass=True, live_slots=slots)
        a1b[layer] = fp.last_mass[layer]
        assert a1b[layer].shape == (1, hkv, live)
        _, mp, lp, _ = OA.splitk_attention(q3, kd2[layer], vd2[layer], k3, v3, mask=mask)
        wmass, _ = OA.prefix_scores(q3, kd2[layer], None, mp, lp, None, list(range(t)), mask=mask,
                                    value_aware=False)
        assert rel_err(a1b[layer], wmass.gather(-1, new_phys[layer])) < 1e-4
        fp.probe(layer, qp2.to(gpu), kp2.to(gpu), vp2.to(gpu), live_slots=slots)
        _, mpp, lpp, _ = OA.splitk_attention(qp2, kd2[layer], vd2[layer], kp2, vp2, causal_block=t, mask=mask)
        wpm, _ = OA.prefix_scores(qp2, kd2[layer], None, mpp, lpp, None, list(range(t, 2 * t)), mask=mask,
                                  value_aware=False)
        assert rel_err(fp.probe_mass[layer], wpm.gather(-1, new_phys[layer])) < 1e-4
    score2 = lookahead_scores(cache, st, a1b, fp.probe_mass, use_value=True)
    for layer in range(L):
        a = (a1b[layer] + fp.probe_mass[layer]).cpu()
        gi = new_phys[layer].unsqueeze(-1).expand(-1, -1, -1, d)
        assert torch.equal(score2[layer].cpu(), OA.value_score_bf16(a, vd2[layer].gather(2, gi)))
    # the same from masses kept per physical slot (step 0 without live_slots), put in live
    # order by lookahead_scores for all layers at once
    a1_slot = {}
    for layer in range(L):
        fp.step0(layer, q3.to(gpu), k3.to(gpu), v3.to(gpu), select=False, topk=1, want_mass=True)
        a1_slot[layer] = fp.last_mass[layer]
        assert a1_slot[layer].shape == (1, hkv, cache.length)
    assert torch.equal(lookahead_scores(cache, st, a1_slot, fp.probe_mass, use_value=True, per_slot=True), score2)
    C2 = 768
    pos1 = st.pos[..., :live].cpu().to(torch.int64)
    # the decode loop's hot path: no order-check or rebuild-status read-back
    keep2 = lookahead_evict(cache, st, cfg, C2, a1b, fp.probe_mass, next_position=n, check=False)
    torch.cuda.synchronize()
    assert torch.equal(keep2.cpu(), OS.keep_select(pos1, score2.cpu(), C2, W))
    assert st.live == C2
    cache.check_rebuild()


def test_lookahead_evict_batch_equals_one_by_one(gpu):
    """lookahead_evict_batch over the sequences of a batch (each with its own cache and
    state; the plans' counts read back once for all of them) leaves every cache, state
    and keep set exactly as lookahead_evict called on each sequence in turn does; a
    sequence whose live set already fits is left alone."""
    from maskahead_amd.runtime.session import lookahead_evict_batch

    L, hkv, d, t, C, W = 2, 4, 128, 32, 512, 64
    cfg = EvictionConfig(policy="lookahead", recent_window=W, capacity_floor=W, compaction="lazy", repack_below=0.5)

    def build(n, seed):
        q, k, v, kc, vc = layer_inputs(b=1, hq=28, hkv=hkv, d=d, n=n, t=t, seed=seed)
        cache = PackedKVCache(num_layers=L, batch_size=1, num_kv_heads=hkv, head_dim=d, max_tokens=1 << 14,
                              quant=QuantizationConfig(), device=gpu)
        cache.begin_append(n)
        for layer in range(L):
            cache.stage_layer(layer, (k + layer).to(torch.bfloat16).to(gpu), v.to(torch.bfloat16).to(gpu))
        cache.commit_append()
        st = EvictionState(num_layers=L, batch_size=1, num_kv_heads=hkv, capacity=n, device=gpu)
        st.append(range(n))
        fp = FastLayerPath(cache=cache, block_size=t, query_indices=list(range(t)))
        for layer in range(L):
            fp.step0(layer, q.to(torch.bfloat16).to(gpu), kc.to(torch.bfloat16).to(gpu),
                     vc.to(torch.bfloat16).to(gpu), select=False, topk=1, want_mass=True)
        return cache, st, dict(fp.last_mass)

    lens = (2000, 3100, 400)                    # the last one already fits the capacity
    one = [build(n, 80 + i) for i, n in enumerate(lens)]
    many = [build(n, 80 + i) for i, n in enumerate(lens)]
    keeps1 = [lookahead_evict(c, s, cfg, C, a1, None, next_position=n, check=False)
              for (c, s, a1), n in zip(one, lens)]
    keeps2 = lookahead_evict_batch([(c, s, a1, None, n) for (c, s, a1), n in zip(many, lens)], cfg, C)
    torch.cuda.synchronize()
    assert keeps1[2] is None and keeps2[2] is None
    for (c1, s1, _), (c2, s2, _), k1, k2 in zip(one, many, keeps1, keeps2):
        c1.check_rebuild()
        c2.check_rebuild()
        assert (k1 is None) == (k2 is None) and (k1 is None or torch.equal(k1, k2))
        assert (c1.length, c1.quantized_length, c1.residual_length, c1.dropped) == \
            (c2.length, c2.quantized_length, c2.residual_length, c2.dropped)
        assert s1.live == s2.live and torch.equal(s1.phys[..., :s1.live], s2.phys[..., :s2.live])
        assert torch.equal(s1.pos[..., :s1.live], s2.pos[..., :s2.live])
        for _, name in STORE:
            a, b = getattr(c1, name), getattr(c2, name)
            cut = c1.quantized_length // 32 if name in ("k_q", "k_scale", "k_zero") else \
                c1.quantized_length if name.startswith("v_") and name != "v_residual" else c1.residual_length
            assert same_bits(a[:, :, :, :cut], b[:, :, :, :cut]), name
