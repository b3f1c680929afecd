"""GPU parity of the one-call step 0 (ma_step0 through kernels.step0.step0_select, what
FastLayerPath.step0 runs for a sparse layer): bit-identical to the same stages called one
by one (splitk_attention, prefix_scores_topk, gather_packed_kv) -- attention output, prefix
statistics, mass, score, read set and gathered K/V -- on packed prefixes with a bf16
residual and dead slots, on a bf16 prefix, with in-order and device selection rows, and
on repeated calls that reuse one layer's buffers at a larger and then a smaller prefix."""

import pytest
import torch

from maskahead_amd.kernels import Step0Buffers, gather_packed_kv, prefix_scores_topk, splitk_attention, step0_select
from maskahead_amd.kernels.splitk import Prefix

from _util import gpu_prefix, layer_inputs, packed_cpu

pytestmark = pytest.mark.gpu


def _case(dev, n, tail, *, dead=False, dense=False, hq=28, hkv=4, t=32, seed=3):
    q, k, v, kc, vc = layer_inputs(hq=hq, hkv=hkv, d=128, n=n + tail, t=t, seed=seed, dtype=torch.bfloat16)
    mask = None
    if dead:
        g = torch.Generator().manual_seed(seed + 1)
        mask = (torch.rand((1, hkv, n + tail), generator=g) > 0.2).to(torch.uint8)
    if dense:
        p = Prefix.dense(k.to(dev), v.to(dev), mask=None if mask is None else mask.to(dev))
    else:
        store, nq = packed_cpu(k[:, :, :n], v[:, :, :n], pad_groups=2, pad_tokens=64)
        p = gpu_prefix(store, nq, dev, kf=k[:, :, n:] if tail else None, vf=v[:, :, n:] if tail else None, mask=mask)
    return q.to(dev), p, kc.to(dev), vc.to(dev)


def _reference(q, p, kc, vc, rows, k, value):
    out, stats = splitk_attention(q, p, kc, vc, want_prefix=True)
    mass, score, idx = prefix_scores_topk(q, p, stats, rows, k, value=value, rank="score" if value else "mass")
    ck, cv = gather_packed_kv(p, idx)
    return out, stats, mass, score, idx, ck, cv


def _check(dev, bufs, ws, q, p, kc, vc, rows, k, value):
    want = _reference(q, p, kc, vc, rows, k, value)
    b, hkv = q.shape[0], kc.shape[1]
    ck = torch.full((b, hkv, k + 7, 128), float("nan"), dtype=torch.bfloat16, device=dev)
    cv = torch.full_like(ck, float("nan"))
    out, stats, mass, score, idx = step0_select(bufs, q, p, kc, vc, rows, k, value=value, out_key=ck[:, :, :k],
                                                out_value=cv[:, :, :k], workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(out, want[0])
    for got, exp in zip(stats[:3], want[1][:3]):
        assert torch.equal(got, exp)
    assert stats[3].vround == want[1][3].vround
    assert torch.equal(mass, want[2])
    assert (score is None) == (want[3] is None) and (score is None or torch.equal(score, want[3]))
    assert torch.equal(idx, want[4])
    assert torch.equal(ck[:, :, :k], want[5]) and torch.equal(cv[:, :, :k], want[6])
    assert torch.isnan(ck[:, :, k:].float()).all()          # nothing written past the read set


@pytest.mark.parametrize("dense", [False, True])
def test_step0_fused_equals_stages(gpu, dense):
    bufs, ws = Step0Buffers(), Step0Buffers()
    q, p, kc, vc = _case(gpu, 4096, 40, dead=True, dense=dense)
    _check(gpu, bufs, ws, q, p, kc, vc, list(range(32)), 512, value=True)
    _check(gpu, bufs, ws, q, p, kc, vc, list(range(32)), 512, value=False)
    rows = torch.tensor([3, 17, 31], dtype=torch.int32, device=gpu)    # device rows, not in order
    _check(gpu, bufs, ws, q, p, kc, vc, rows, 700, value=True)


def test_step0_fused_reuses_buffers(gpu):
    bufs, ws = Step0Buffers(), Step0Buffers()
    q, p, kc, vc = _case(gpu, 8192, 0, seed=5)
    _check(gpu, bufs, ws, q, p, kc, vc, list(range(32)), 1024, value=True)
    kept = bufs._store["mass"].data_ptr()
    q2, p2, kc2, vc2 = _case(gpu, 2048, 32, dead=True, seed=6)   # smaller prefix: the same storage
    _check(gpu, bufs, ws, q2, p2, kc2, vc2, list(range(32)), 256, value=True)
    assert bufs._store["mass"].data_ptr() == kept
    q3, p3, kc3, vc3 = _case(gpu, 512, 0, hq=28, hkv=4, t=8, seed=7)  # T = 8 (the Fast-dLLM block cache)
    _check(gpu, bufs, ws, q3, p3, kc3, vc3, list(range(8)), 128, value=True)


def test_step0_fused_repeat_calls(gpu):
    """A layer's repeated step 0 with new operands (same shapes, the same prefix object,
    rows and output views): the call reuses its checked arguments and gives the stages'
    results every time; a change of read budget re-plans."""
    bufs, ws = Step0Buffers(), Step0Buffers()
    _, p, _, _ = _case(gpu, 4096, 40, dead=True, seed=11)
    b, hkv, k = 1, 4, 512
    ck = torch.empty((b, hkv, 1024, 128), dtype=torch.bfloat16, device=gpu)
    cv = torch.empty_like(ck)
    plans = []
    for i, kk in enumerate((k, k, k, 300)):
        q, _, kc, vc = _case(gpu, 4096, 40, dead=True, seed=20 + i)
        want = _reference(q, p, kc, vc, list(range(32)), kk, True)
        out, stats, mass, score, idx = step0_select(bufs, q, p, kc, vc, list(range(32)), kk, value=True,
                                                    out_key=ck[:, :, :kk], out_value=cv[:, :, :kk], workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(out, want[0]) and torch.equal(mass, want[2]) and torch.equal(score, want[3])
        assert torch.equal(idx, want[4])
        assert torch.equal(ck[:, :, :kk], want[5]) and torch.equal(cv[:, :, :kk], want[6])
        plans.append(bufs._plan[4])
    assert plans[0] is plans[1] is plans[2] and plans[3] is not plans[2]


def test_step0_fused_errors(gpu):
    bufs = Step0Buffers()
    q, p, kc, vc = _case(gpu, 1024, 0, seed=8)
    with pytest.raises(ValueError):
        step0_select(bufs, q, p, kc, vc, list(range(32)), 0, value=True)
    with pytest.raises(ValueError):
        step0_select(bufs, q, p, kc, vc, list(range(32)), 2000, value=True)
    with pytest.raises(ValueError):
        step0_select(bufs, q, p, kc, vc, [40], 10, value=True)
