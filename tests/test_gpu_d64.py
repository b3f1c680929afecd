"""head_dim 64, which the fast path serves (fast_path_supported) besides 128: the one-call
step 0 over a packed prefix with a bf16 residual and dead slots -- attention, prefix
statistics, mass and value score against the oracle, the read set against the oracle's
top-k of the same scores, the gathered entries against the oracle's dequantization -- and
a sub-step over the gathered read set against the oracle's attention."""

import pytest
import torch

from maskahead_amd.kernels import Step0Buffers, step0_select
from maskahead_amd.kernels.splitk import Prefix, splitk_attention
from oracle import attention as OA
from oracle import selection as OS

from _util import assert_attention_close, dequant_cpu, gpu_prefix, layer_inputs, packed_cpu, rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dense", [False, True])
def test_step0_and_substep_head_dim_64(gpu, dense):
    n, tail, hq, hkv, d, t, k = 3072, 24, 16, 4, 64, 32, 384
    q, kk, v, kc, vc = layer_inputs(hq=hq, hkv=hkv, d=d, n=n + tail, t=t, seed=81, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(82)
    mask = (torch.rand((1, hkv, n + tail), generator=g) > 0.15).to(torch.uint8)
    if dense:
        kd, vd = kk, v
        p = Prefix.dense(kk.to(gpu), v.to(gpu), mask=mask.to(gpu))
    else:
        store, nq = packed_cpu(kk[:, :, :n], v[:, :, :n], pad_groups=1, pad_tokens=32)
        p = gpu_prefix(store, nq, gpu, kf=kk[:, :, n:], vf=v[:, :, n:], mask=mask)
        kq, vq = dequant_cpu(store, nq)
        kd = torch.cat([kq.to(torch.bfloat16), kk[:, :, n:]], 2)
        vd = torch.cat([vq.to(torch.bfloat16), v[:, :, n:]], 2)
    qg, kcg, vcg = q.to(gpu), kc.to(gpu), vc.to(gpu)
    ck = torch.empty((1, hkv, k, d), dtype=torch.bfloat16, device=gpu)
    cv = torch.empty_like(ck)
    out, stats, mass, score, idx = step0_select(Step0Buffers(), qg, p, kcg, vcg, list(range(t)), k, value=True,
                                                out_key=ck, out_value=cv)
    torch.cuda.synchronize()
    wout, wmp, wlp, wop = OA.splitk_attention(q, kd, vd, kc, vc, mask=mask)
    assert_attention_close(out, wout)
    assert rel_err(stats[0].cpu()[wmp > -1e30], wmp[wmp > -1e30]) < 1e-5
    assert rel_err(stats[1], wlp) < 1e-4
    mp, lp, op = (x.cpu() for x in stats[:3])
    # the value distance reads V as the reference's unpacked bf16 copy (n > 256)
    wmass, wscore = OA.prefix_scores(q, kd, vd.float(), mp, lp, op, list(range(t)), mask=mask, value_aware=True)
    live = mask.bool()
    assert torch.all(mass.cpu()[~live] == 0)
    assert rel_err(mass.cpu()[live], wmass[live]) < 2e-5
    assert rel_err(score.cpu()[live], wscore[live]) < 2e-5
    assert torch.equal(idx.cpu(), OS.topk_ascending(score.cpu(), k, mask))
    gi = idx.cpu().unsqueeze(-1).expand(-1, -1, -1, d)
    assert torch.equal(ck.cpu(), kd.gather(2, gi)) and torch.equal(cv.cpu(), vd.gather(2, gi))
    # a sub-step over [read set | block]
    q2 = torch.randn((1, hq, t, d), generator=g).to(torch.bfloat16)
    o2, _ = splitk_attention(q2.to(gpu), Prefix.dense(ck, cv), kcg, vcg)
    assert_attention_close(o2, OA.dense_attention(q2, ck.cpu(), cv.cpu(), kc, vc))
