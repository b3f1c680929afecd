"""The oracle's floating-point half (oracle/attention.py) pinned by textbook routines
(torch SDPA, softmax), closed-form identities and brute force on tiny inputs."""

import math

import pytest
import torch
import torch.nn.functional as F

from maskahead_amd.workloads import layer_inputs
from oracle import attention as OA

F64 = torch.float64


def _bf(x):
    return x.to(torch.bfloat16).to(F64)


def _sdpa(q, k, v, mask=None):
    g = q.shape[1] // k.shape[1]
    return F.scaled_dot_product_attention(q, k.repeat_interleave(g, 1), v.repeat_interleave(g, 1),
                                          attn_mask=mask)


def test_splitk_matches_sdpa_and_prefix_stats():
    q, k, v, kc, vc = layer_inputs(hq=8, hkv=2, d=64, n=200, t=16, seed=7)
    out, mp, lp, op = OA.splitk_attention(q, k, v, kc, vc)
    qb, kb, vb, kcb, vcb = (_bf(x) for x in (q, k, v, kc, vc))
    want = _sdpa(qb, torch.cat([kb, kcb], 2), torch.cat([vb, vcb], 2))
    assert torch.allclose(out.to(F64), want, rtol=1e-5, atol=1e-6)
    # prefix-only statistics: softmax over the prefix alone
    want_p = _sdpa(qb, kb, vb).reshape(1, 2, 4 * 16, 64)
    assert torch.allclose(op.to(F64), want_p, rtol=1e-5, atol=1e-6)
    s = torch.matmul(qb.reshape(1, 2, 64, 64), kb.transpose(-1, -2)) / 8.0
    assert torch.allclose(mp.to(F64), s.amax(-1), rtol=1e-6)
    assert torch.allclose(lp.to(F64), torch.exp(s - s.amax(-1, keepdim=True)).sum(-1), rtol=1e-5)


def test_lse_merge_identity():
    # merging the prefix statistics with the current block's reproduces the output
    q, k, v, kc, vc = layer_inputs(hq=4, hkv=1, d=64, n=96, t=8, seed=8)
    out, mp, lp, op = OA.splitk_attention(q, k, v, kc, vc)
    qb, kcb, vcb = _bf(q).reshape(1, 1, 32, 64), _bf(kc), _bf(vc)
    sc = torch.matmul(qb, kcb.transpose(-1, -2)) / 8.0
    mc = sc.amax(-1)
    lc = torch.exp(sc - mc.unsqueeze(-1)).sum(-1)
    oc = torch.softmax(sc, -1) @ vcb
    m = torch.maximum(mp.to(F64), mc)
    wp, wc = lp.to(F64) * torch.exp(mp.to(F64) - m), lc * torch.exp(mc - m)
    merged = (op.to(F64) * wp.unsqueeze(-1) + oc * wc.unsqueeze(-1)) / (wp + wc).unsqueeze(-1)
    assert torch.allclose(merged.reshape(out.shape), out.to(F64), rtol=1e-5, atol=1e-6)


def test_dead_slots_equal_dropping_them():
    q, k, v, kc, vc = layer_inputs(hq=4, hkv=2, d=64, n=64, t=4, seed=9)
    g = torch.Generator().manual_seed(0)
    mask = (torch.rand((1, 2, 64), generator=g) > 0.4).to(torch.uint8)
    out, mp, lp, op = OA.splitk_attention(q, k, v, kc, vc, mask=mask)
    for h in range(2):
        live = mask[0, h].bool()
        o_h, _, _, op_h = OA.splitk_attention(q[:, 2 * h:2 * h + 2], k[:, h:h + 1, live], v[:, h:h + 1, live],
                                              kc[:, h:h + 1], vc[:, h:h + 1])
        assert torch.equal(o_h, out[:, 2 * h:2 * h + 2])
        assert torch.allclose(op_h[0, 0], op[0, h])


def test_block_causal_brute_force():
    q, k, v, kc, vc = layer_inputs(hq=2, hkv=1, d=64, n=32, t=12, seed=10)
    cb, qp0, cp0 = 4, 5, 5
    out, *_ = OA.splitk_attention(q, k, v, kc, vc, causal_block=cb, q_pos0=qp0, c_pos0=cp0)
    allowed = torch.zeros((12, 32 + 12), dtype=torch.bool)
    for t in range(12):
        for j in range(32 + 12):
            allowed[t, j] = j < 32 or (cp0 + j - 32) // cb <= (qp0 + t) // cb
    want = _sdpa(_bf(q), torch.cat([_bf(k), _bf(kc)], 2), torch.cat([_bf(v), _bf(vc)], 2),
                 mask=allowed[None, None])
    assert torch.allclose(out.to(F64), want, rtol=1e-5, atol=1e-6)


def test_mass_equals_selector_importance():
    q, k, v, kc, vc = layer_inputs(hq=8, hkv=2, d=64, n=128, t=16, seed=11)
    mask = torch.ones((1, 2, 128), dtype=torch.uint8)
    mask[0, 1, ::5] = 0
    _, mp, lp, op = OA.splitk_attention(q, k, v, kc, vc, mask=mask)
    rows = [1, 4, 5, 9, 15]
    mass, score = OA.prefix_scores(q, k, v, mp, lp, op, rows, mask=mask, value_aware=True)
    imp = OA.selector_importance(_bf(q), _bf(k), rows, live_mask=mask)
    assert torch.allclose(mass.to(F64), imp, rtol=1e-5, atol=1e-12)
    assert torch.allclose(mass.sum(-1).to(F64), torch.ones(1, 2, dtype=F64), rtol=1e-5)
    # value score against the torch path's centre (session.py:870-954): c = sum a v / sum a;
    # the fast path's centre is the mean of O_p (whose PV product reads bf16 V) in the
    # query dtype -- equal here, f32 queries keep O_p in f32 -- and the distance reads the
    # prefix V as given (f32 here, splitk.py:364-369)
    vv = _bf(v)
    c = (mass.to(F64).unsqueeze(-1) * vv).sum(2, keepdim=True) / mass.to(F64).sum(-1, keepdim=True).unsqueeze(-1)
    want = mass.to(F64) * (v.to(F64) - c).norm(dim=-1)
    assert torch.allclose(score.to(F64), want * mask, rtol=1e-4, atol=1e-9)
    assert torch.all(score[mask == 0] == 0) and torch.all(mass[mask == 0] == 0)


def test_value_score_fp32_vs_bf16_branch():
    g = torch.Generator().manual_seed(12)
    a = torch.rand((1, 2, 300), generator=g) / 300
    v = torch.randn((1, 2, 300, 128), generator=g).to(torch.bfloat16)
    s16 = OA.value_score_bf16(a, v)
    s32 = OA.value_score_fp32(a, v)
    assert torch.allclose(s16, s32, rtol=2e-2)


def test_dense_attention_matches_sdpa_and_brute_force():
    """oracle.dense_attention (reference.py:279-315, the sub-step's sdpa_compact) against
    torch's SDPA with the KV heads repeated per GQA group, and against an explicit
    per-(head, query) softmax loop on a tiny case."""
    q, k, v, kc, vc = layer_inputs(hq=12, hkv=3, d=32, n=50, t=6, seed=17, dtype=F64)
    got = OA.dense_attention(q, k, v, kc, vc)
    want = _sdpa(q, torch.cat([k, kc], 2), torch.cat([v, vc], 2))
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)
    # brute force: head h reads KV head h // 4; one softmax per query row
    kk, vv = torch.cat([k, kc], 2), torch.cat([v, vc], 2)
    for h in (0, 5, 11):
        for t in (0, 5):
            s = torch.tensor([float((q[0, h, t] * kk[0, h // 4, j]).sum()) / math.sqrt(32) for j in range(56)],
                             dtype=F64)
            w = torch.exp(s - s.max())
            o = (w[:, None] * vv[0, h // 4]).sum(0) / w.sum()
            assert torch.allclose(got[0, h, t], o, rtol=1e-12, atol=1e-12)
    # a custom scale enters the logits only
    half = OA.dense_attention(q, k, v, kc, vc, scale=0.5 / math.sqrt(32))
    assert torch.allclose(half, OA.dense_attention(q * 0.5, k, v, kc, vc), rtol=1e-12, atol=1e-12)
