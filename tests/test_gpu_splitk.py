"""GPU parity, split-K attention (splitk.py:493-579): the output within the north-star
tolerance (2e-2 abs / 1e-2 rel) of the CPU oracle, and the prefix statistics M_p, L_p,
O_p (which feed the scores) much tighter."""

import pytest
import torch

from maskahead_amd.kernels.splitk import Prefix, splitk_attention
from oracle import attention as OA

from _util import assert_attention_close, dequant_cpu, gpu_prefix, layer_inputs, packed_cpu, rel_err

pytestmark = pytest.mark.gpu


def _check_stats(gpu_stats, want):
    mp, lp, op = (x.cpu() for x in gpu_stats[:3])
    _, wmp, wlp, wop = want
    fin = torch.isfinite(wmp)
    assert torch.equal(torch.isfinite(mp), fin)
    assert rel_err(mp[fin], wmp[fin]) < 1e-5
    assert rel_err(lp[fin], wlp[fin]) < 1e-4          # f32 sums of exp; bf16(p) only enters O
    assert_attention_close(op, wop, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("split_tokens", [0, 256, 1024])
def test_config0_fp32_dense_prefix(gpu, split_tokens):
    # BASELINE config 0 shape: 28/4 heads, D 128, prefix 4096, block 32, fp32 inputs
    q, k, v, kc, vc = layer_inputs(hq=28, hkv=4, d=128, n=4096, t=32, seed=1234)
    want = OA.splitk_attention(q, k, v, kc, vc)
    p = Prefix.dense(k.to(gpu), v.to(gpu))
    out, stats = splitk_attention(q.to(gpu), p, kc.to(gpu), vc.to(gpu), want_prefix=True, split_tokens=split_tokens)
    assert out.dtype == torch.float32
    assert_attention_close(out, want[0])
    _check_stats(stats, want)


def test_packed_prefix_with_residual_and_mask(gpu):
    q, k, v, kc, vc = layer_inputs(hq=28, hkv=4, d=128, n=2048 + 24, t=32, seed=3, dtype=torch.bfloat16)
    store, nq = packed_cpu(k[:, :, :2048], v[:, :, :2048], pad_groups=5, pad_tokens=100)
    kt, vt = k[:, :, 2048:], v[:, :, 2048:]
    g = torch.Generator().manual_seed(4)
    mask = (torch.rand((1, 4, 2048 + 24), generator=g) > 0.3).to(torch.uint8)
    mask[:, :, :4] = 1
    p = gpu_prefix(store, nq, gpu, kf=kt, vf=vt, mask=mask)
    out, stats = splitk_attention(q.to(gpu), p, kc.to(gpu), vc.to(gpu), want_prefix=True)
    kd, vd = dequant_cpu(store, nq)
    want = OA.splitk_attention(q, torch.cat([kd, kt.float()], 2), torch.cat([vd, vt.float()], 2), kc, vc, mask=mask)
    assert out.dtype == torch.bfloat16
    assert_attention_close(out, want[0])
    _check_stats(stats, want)


def test_block_causal_current_and_positions(gpu):
    # probe-style call: 3 blocks of 32 queries, block-causal over the current tokens
    q, k, v, kc, vc = layer_inputs(hq=8, hkv=2, d=128, n=512, t=96, seed=5, dtype=torch.bfloat16)
    want = OA.splitk_attention(q, k, v, kc, vc, causal_block=32, q_pos0=64, c_pos0=64)
    out, _ = splitk_attention(q.to(gpu), Prefix.dense(k.to(gpu), v.to(gpu)), kc.to(gpu), vc.to(gpu),
                              causal_block=32, q_pos0=64, c_pos0=64)
    assert_attention_close(out, want[0])


def test_row_groups_and_head_dim_64(gpu):
    # G = 4, T = 96 -> R = 384 rows per KV head (two row groups); D = 64
    q, k, v, kc, vc = layer_inputs(hq=16, hkv=4, d=64, n=1000, t=96, seed=6, dtype=torch.bfloat16)
    want = OA.splitk_attention(q, k, v, kc, vc)
    out, stats = splitk_attention(q.to(gpu), Prefix.dense(k.to(gpu), v.to(gpu)), kc.to(gpu), vc.to(gpu),
                                  want_prefix=True)
    assert_attention_close(out, want[0])
    _check_stats(stats, want)


def test_empty_prefix_and_all_dead(gpu):
    q, k, v, kc, vc = layer_inputs(hq=4, hkv=2, d=128, n=64, t=8, seed=7, dtype=torch.bfloat16)
    empty = Prefix()
    out, _ = splitk_attention(q.to(gpu), empty, kc.to(gpu), vc.to(gpu))
    want = OA.splitk_attention(q, k[:, :, :0], v[:, :, :0], kc, vc)
    assert_attention_close(out, want[0])
    dead = torch.zeros((1, 2, 64), dtype=torch.uint8)
    out2, stats = splitk_attention(q.to(gpu), Prefix.dense(k.to(gpu), v.to(gpu), mask=dead.to(gpu)), kc.to(gpu),
                                   vc.to(gpu), want_prefix=True)
    assert_attention_close(out2, want[0])
    assert torch.all(torch.isneginf(stats[0].cpu())) and torch.all(stats[1].cpu() == 0)
    assert torch.all(stats[2].cpu() == 0)
