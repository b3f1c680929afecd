"""GPU parity of the operator API a session binds (kernels/ops.py:130-264, 333-521, 766-832;
kernels/splitk.py:493-614) and of the per-layer routing of the fast path
(session.py:2281-2418, 456-467): selector_topk, dense_packed_attention and the value
centre against the oracle; the score pass's rounding of packed values to the query dtype;
probe and prefill-chunk shapes beyond 512 selection rows; one whole block of a 4-layer
model (2 dense + 2 sparse layers) routed call by call."""

from __future__ import annotations

import ctypes

import pytest
import torch

from maskahead_amd import _native as N
from maskahead_amd.cache import PackedKVCache
from maskahead_amd.config import QuantizationConfig
from maskahead_amd.kernels.ops import _selected_queries, dense_packed_attention, selector_topk
from maskahead_amd.kernels.select import prefix_scores_topk
from maskahead_amd.kernels.splitk import Prefix, prefix_scores, splitk_attention
from maskahead_amd.kernels.step0 import Step0Buffers, step0_select
from maskahead_amd.runtime.fastpath import BlockContext, FastLayerPath
from maskahead_amd.workloads import layer_inputs
from oracle import attention as OA
from oracle import selection as OS

from _util import assert_attention_close, dequant_cpu, gpu_prefix, packed_cpu, rel_err

pytestmark = pytest.mark.gpu

BF16 = QuantizationConfig(k_bits=16, v_bits=16)


def _cache(gpu, k, v, quant, layers=1, extra=64):
    """A cache holding [B,H,n,D] K/V in every layer (layer l: K + l), and the oracle's
    view of each layer (bf16, dequantized where packed)."""
    b, h, n, d = k.shape
    c = PackedKVCache(num_layers=layers, batch_size=b, num_kv_heads=h, head_dim=d, max_tokens=n + extra,
                      quant=quant, device=gpu)
    c.begin_append(n)
    for layer in range(layers):
        c.stage_layer(layer, (k + layer).to(torch.bfloat16).to(gpu), v.to(torch.bfloat16).to(gpu))
    c.commit_append()
    views = [tuple(x.cpu() for x in c.dequantize_layer(layer)) for layer in range(layers)]
    return c, views


@pytest.mark.parametrize("packed", [False, True])
def test_selector_topk_against_oracle(gpu, packed):
    """selector_topk (ops.py:333-521, domain prefix, score softmax): the importance is the
    mean prefix-softmax of the selection queries with dead entries removed; the read set
    its top-k, ascending; values = importance at those indices."""
    n, t, topk = 3000, 32, 300
    q, k, v, _, _ = layer_inputs(b=1, hq=28, hkv=4, d=128, n=n, t=t, seed=51)
    c, views = _cache(gpu, k, v, QuantizationConfig() if packed else BF16)
    kd = views[0][0]
    live = torch.rand((1, 4, n), generator=torch.Generator().manual_seed(52)) > 0.1
    live[:, :, :4] = True
    rows = [0, 5, 17, 31]
    qb = q.to(torch.bfloat16)
    res = selector_topk(qb.to(gpu), c.layer_view(0), query_indices=rows, topk=topk, live_mask=live.to(gpu),
                        return_importance=True)
    want = OA.selector_importance(qb.float(), kd.float(), rows, live_mask=live)
    err = rel_err(res.importance[live.to(gpu)], want[live])
    assert err < 2e-3
    # the read set against the oracle's importance: members may differ only inside the
    # band the measured importance error allows at the k-th value
    ok, nmis, worst = OS.boundary_mismatch_ok(res.indices.cpu(), OS.topk_ascending(want.float(), topk, live),
                                              want, topk, rel=2 * err + 1e-6, mask=live)
    assert ok, (nmis, worst, err)
    assert bool(torch.all(live.gather(2, res.indices.cpu())))
    assert torch.equal(res.values.cpu(), res.importance.cpu().gather(2, res.indices.cpu()))
    # _selected_queries: the selection rows of each KV head, r = g * T2 + t2 (ops.py:320-330)
    sq = _selected_queries(qb, rows, 4)
    assert sq.shape == (1, 4, 7 * len(rows), 128)
    assert torch.equal(sq[0, 1, 2 * len(rows) + 1], qb[0, 1 * 7 + 2, rows[1]])


@pytest.mark.parametrize("packed", [False, True])
def test_dense_packed_attention_against_oracle(gpu, packed):
    """dense_packed_attention (ops.py:766-787): softmax attention over [cache | block]."""
    q, k, v, kc, vc = layer_inputs(b=1, hq=28, hkv=4, d=128, n=2500, t=32, seed=53, dtype=torch.bfloat16)
    c, views = _cache(gpu, k, v, QuantizationConfig() if packed else BF16)
    out = dense_packed_attention(q.to(gpu), c.layer_view(0), kc.to(gpu), vc.to(gpu))
    assert_attention_close(out, OA.dense_attention(q, views[0][0], views[0][1], kc, vc))


def test_value_centre_against_oracle(gpu):
    """ma_value_centre (splitk.py:599-601): the mean over the G * T2 selection rows of
    f32(O_p); repeated block positions count once per occurrence."""
    lib = N.load()
    g = torch.Generator().manual_seed(54)
    b, h, gq, t, d = 1, 4, 7, 32, 128
    op = (torch.randn((b, h, gq * t, d), generator=g) * 3).to(torch.bfloat16)
    rows = [0, 3, 3, 31, 17]
    centre = torch.empty((b, h, d), device=gpu)
    qr = torch.tensor(rows, dtype=torch.int32, device=gpu)
    N.check(lib.ma_value_centre(op.to(gpu).data_ptr(), N.MA_BF16, b, h, gq, t, d, qr.data_ptr(), len(rows),
                                centre.data_ptr(), N.stream_of(centre)), "ma_value_centre")
    rf = (torch.arange(gq)[:, None] * t + torch.tensor(rows)[None, :]).reshape(-1)
    want = op[:, :, rf].double().mean(2)
    assert rel_err(centre, want) < 1e-6


def test_f16_queries_read_an_f16_copy_of_a_packed_prefix(gpu):
    """A packed prefix longer than packed_direct_max is read by the reference through a copy
    unpacked to the query dtype (splitk.py:513-516): with f16 queries K and V are rounded
    f32 -> f16 into that copy and f16 -> bf16 at every dot, and the value distance sees the
    f16 values.  The copy is bit-identical to the oracle's dequantization rounded to f16;
    attention, statistics, scores and the step-0 call follow it.  The caller's Prefix is
    left as it was."""
    q, k, v, kc, vc = layer_inputs(b=1, hq=28, hkv=4, d=128, n=1024, t=32, seed=55)
    store, nq = packed_cpu(k.to(torch.bfloat16), v.to(torch.bfloat16))
    pre = gpu_prefix(store, nq, gpu)
    qh, kch, vch = q.to(torch.float16), kc.to(torch.float16), vc.to(torch.float16)
    out, stats = splitk_attention(qh.to(gpu), pre, kch.to(gpu), vch.to(gpu), want_prefix=True)
    used = stats[3]
    assert pre.vround == 0 and pre.nq == nq and used.nq == 0 and used.kf.dtype == torch.float16
    kd, vd = dequant_cpu(store, nq)
    kd16, vd16 = kd.to(torch.float16), vd.to(torch.float16)
    assert torch.equal(used.kf.cpu(), kd16) and torch.equal(used.vf.cpu(), vd16)
    wout, wmp, wlp, wop = OA.splitk_attention(qh, kd16, vd16, kch, vch)
    assert_attention_close(out, wout)
    assert rel_err(stats[0], wmp) < 1e-5 and rel_err(stats[1], wlp) < 1e-4
    # the bar has teeth: rounding K and V to bf16 once gives statistics outside it
    _, smp, slp, _ = OA.splitk_attention(qh, kd, vd, kch, vch)
    assert rel_err(smp, wmp) > 1e-4 or rel_err(slp, wlp) > 1e-3
    mass, score = prefix_scores(qh.to(gpu), pre, stats, torch.arange(32, dtype=torch.int32), value=True)
    mp, lp, op = (x.cpu() for x in stats[:3])
    wmass, wscore = OA.prefix_scores(qh, kd16, vd16.float(), mp, lp, op, range(32), value_aware=True)
    assert rel_err(mass, wmass) < 1e-4
    assert rel_err(score, wscore) < 1e-4
    # the one-call step 0 gives the same (it runs the stages for this case)
    ck = torch.empty((1, 4, 256, 128), dtype=torch.float16, device=gpu)
    cv = torch.empty_like(ck)
    out2, stats2, mass2, score2, idx2 = step0_select(Step0Buffers(), qh.to(gpu), pre, kch.to(gpu), vch.to(gpu),
                                                     list(range(32)), 256, value=True, out_key=ck, out_value=cv)
    _, _, widx = prefix_scores_topk(qh.to(gpu), pre, stats, list(range(32)), 256, value=True)
    assert torch.equal(out2, out) and torch.equal(mass2, mass) and torch.equal(score2, score)
    assert torch.equal(idx2, widx)
    gi = widx.cpu().unsqueeze(-1).expand(-1, -1, -1, 128)
    assert torch.equal(ck.cpu(), kd16.gather(2, gi)) and torch.equal(cv.cpu(), vd16.gather(2, gi))


def test_mask_of_the_wrong_shape_is_rejected(gpu):
    """The kernels index the slot mask as [B, Hkv, n]; a broadcastable [1, Hkv, n] mask for
    a batch of 2 is a ValueError before any launch."""
    q, k, v, kc, vc = layer_inputs(b=2, hq=8, hkv=2, d=128, n=256, t=8, seed=56, dtype=torch.bfloat16)
    bad = torch.ones((1, 2, 256), dtype=torch.uint8, device=gpu)
    pre = Prefix.dense(k.to(gpu), v.to(gpu), mask=bad)
    with pytest.raises(ValueError, match="mask"):
        splitk_attention(q.to(gpu), pre, kc.to(gpu), vc.to(gpu))


def test_probe_of_four_blocks_and_long_prefill_chunk(gpu):
    """A lookahead probe of 4 masked blocks (t = 128: 7 x 96 = 672 selection rows per KV
    head) and a 512-token prefill chunk with its mass (7 x 512 = 3 584 rows per KV head):
    the mass runs in passes of at most 512 rows."""
    n, d, blk = 1024, 128, 32
    q, k, v, kc, vc = layer_inputs(b=1, hq=28, hkv=4, d=d, n=n, t=512, seed=57, dtype=torch.bfloat16)
    c, views = _cache(gpu, k, v, QuantizationConfig())
    kd, vd = views[0]
    fp = FastLayerPath(cache=c, block_size=blk, query_indices=list(range(blk)))
    qp, kp, vp = q[:, :, :128], kc[:, :, :128], vc[:, :, :128]
    out = fp.probe(0, qp.to(gpu), kp.to(gpu), vp.to(gpu))
    wout, mp, lp, _ = OA.splitk_attention(qp, kd, vd, kp, vp, causal_block=blk)
    assert_attention_close(out, wout)
    wmass, _ = OA.prefix_scores(qp, kd, None, mp, lp, None, list(range(blk, 128)), value_aware=False)
    assert rel_err(fp.probe_mass[0], wmass * 3) < 1e-4
    out = fp.prefill_chunk(0, q.to(gpu), kc.to(gpu), vc.to(gpu), want_mass=True)
    wout, mp, lp, _ = OA.splitk_attention(q, kd, vd, kc, vc, causal_block=blk)
    assert_attention_close(out, wout)
    wmass, _ = OA.prefix_scores(q, kd, None, mp, lp, None, list(range(512)), value_aware=False)
    assert rel_err(fp.chunk_mass[0], wmass) < 1e-4


def test_route_one_block_of_a_four_layer_model(gpu):
    """One block of a 4-layer model through FastLayerPath.route, as the session's attend
    hook sends each call: layers 0-1 dense (dense_prefix_layers = 2), layers 2-3 sparse.
    Step 0 (sparse layers select 256 of 2 048 by value-aware score), 3 sub-steps (dense
    layers over the prefix, sparse layers over their read set), a lookahead probe of 2
    blocks and a prefill chunk; every output against the oracle."""
    L, hq, hkv, d, n, t, topk = 4, 28, 4, 128, 2048, 32, 256
    q, k, v, kc, vc = layer_inputs(b=1, hq=hq, hkv=hkv, d=d, n=n, t=t, seed=58, dtype=torch.bfloat16)
    c, views = _cache(gpu, k, v, QuantizationConfig(), layers=L)
    fp = FastLayerPath(cache=c, block_size=t, query_indices=list(range(t)), dense_prefix_layers=2)
    ctx = BlockContext(step_index=0, old_cache_len=n, topk=topk)
    assert [fp.dense_required(layer, ctx) for layer in range(L)] == [True, True, False, False]
    for layer in range(L):
        kd, vd = views[layer]
        out = fp.route(layer, q.to(gpu), kc.to(gpu), vc.to(gpu), ctx)
        wout, mp, lp, op = OA.splitk_attention(q, kd, vd, kc, vc)
        assert_attention_close(out, wout)
        if layer < 2:
            assert layer not in fp.states                  # dense layers select nothing
            continue
        # the read set against oracle scores from the GPU's own statistics (the same
        # deterministic pass 1 step 0 ran): members may differ only inside the band the
        # measured score error allows at the k-th value
        pre = fp.prefix(layer)
        _, st = splitk_attention(q.to(gpu), pre, kc.to(gpu), vc.to(gpu), want_prefix=True)
        _, gscore = prefix_scores(q.to(gpu), pre, st, torch.arange(t, dtype=torch.int32), value=True)
        gmp, glp, gop = (x.cpu() for x in st[:3])
        _, wscore = OA.prefix_scores(q, kd, vd.float(), gmp, glp, gop, range(t), value_aware=True)
        err = rel_err(gscore, wscore)
        assert err < 1e-4
        idx = fp.states[layer].indices.cpu()
        ok, nmis, worst = OS.boundary_mismatch_ok(idx, OS.topk_ascending(wscore, topk), wscore, topk,
                                                  rel=2 * err + 1e-6)
        assert ok, (layer, nmis, worst, err)
    g = torch.Generator().manual_seed(59)
    for step in (1, 2, 3):
        ctx.step_index = step
        q2 = torch.randn((1, hq, t, d), generator=g).to(torch.bfloat16)
        k2 = torch.randn((1, hkv, t, d), generator=g).to(torch.bfloat16)
        v2 = torch.randn((1, hkv, t, d), generator=g).to(torch.bfloat16)
        for layer in range(L):
            kd, vd = views[layer]
            out = fp.route(layer, q2.to(gpu), k2.to(gpu), v2.to(gpu), ctx)
            if layer < 2:
                want = OA.dense_attention(q2, kd, vd, k2, v2)
            else:
                gi = fp.states[layer].indices.cpu().unsqueeze(-1).expand(-1, -1, -1, d)
                want = OA.dense_attention(q2, kd.gather(2, gi), vd.gather(2, gi), k2, v2)
            assert_attention_close(out, want)
    # a lookahead probe of the next 2 blocks, then a prefill chunk of 64 tokens
    probe = BlockContext(probe=True, old_cache_len=n, topk=topk)
    qp = torch.randn((1, hq, 2 * t, d), generator=g).to(torch.bfloat16)
    kp = torch.randn((1, hkv, 2 * t, d), generator=g).to(torch.bfloat16)
    vp = torch.randn((1, hkv, 2 * t, d), generator=g).to(torch.bfloat16)
    chunk = BlockContext(prefill=True, want_mass=True)
    for layer in range(L):
        kd, vd = views[layer]
        out = fp.route(layer, qp.to(gpu), kp.to(gpu), vp.to(gpu), probe)
        wout, mp, lp, _ = OA.splitk_attention(qp, kd, vd, kp, vp, causal_block=t)
        assert_attention_close(out, wout)
        wmass, _ = OA.prefix_scores(qp, kd, None, mp, lp, None, list(range(t, 2 * t)), value_aware=False)
        assert rel_err(fp.probe_mass[layer], wmass) < 1e-4
        out = fp.route(layer, qp.to(gpu), kp.to(gpu), vp.to(gpu), chunk)
        assert_attention_close(out, wout)
        wmass, _ = OA.prefix_scores(qp, kd, None, mp, lp, None, list(range(2 * t)), value_aware=False)
        assert rel_err(fp.chunk_mass[layer], wmass) < 1e-4
