"""BASELINE config 0 as one fp32 workload on the GPU (the reference's CPU-runnable check:
28/4 heads, D 128, fp32 prefix of 4096, block 32, read budget 512, keep budget 1024):
split-K attention with its prefix statistics, the prefix mass of the 32 block positions
(the selector importance, reference.py:318-366), the read set of 512 per KV head on that
mass (session.py:1429-1438) and the keep set of 1024 on it (eviction.py:325-409: the 128
newest kept outright, the rest by rank) -- each stage on the GPU's own outputs, checked
against the CPU oracle: attention within the north star's tolerance, the mass within 2e-5
of the oracle's from the same statistics, the read and keep sets bit-exact against the
oracle's selection of the GPU's mass and, end to end, differing only at the boundary."""

import torch

import pytest

from maskahead_amd.kernels import prefix_scores, splitk_attention, topk_ascending
from maskahead_amd.kernels.keep import keep_select
from maskahead_amd.kernels.splitk import Prefix
from oracle import attention as OA
from oracle import selection as OS

from _util import assert_attention_close, check_read_set, layer_inputs, rel_err

pytestmark = pytest.mark.gpu

READ, KEEP, WINDOW = 512, 1024, 128


def test_config0_fp32_workload(gpu):
    q, k, v, kc, vc = layer_inputs(hq=28, hkv=4, d=128, n=4096, t=32, seed=1234)
    n = k.shape[2]
    p = Prefix.dense(k.to(gpu), v.to(gpu))
    qg = q.to(gpu)
    out, stats = splitk_attention(qg, p, kc.to(gpu), vc.to(gpu), want_prefix=True)
    wout, wmp, wlp, wop = OA.splitk_attention(q, k, v, kc, vc)
    assert out.dtype == torch.float32
    assert_attention_close(out, wout)

    rows = list(range(32))
    mass, none = prefix_scores(qg, p, stats, torch.tensor(rows, dtype=torch.int32), value=False)
    assert none is None
    gmp, glp, gop = (x.cpu() for x in stats[:3])
    smass, _ = OA.prefix_scores(q, k, None, gmp, glp, gop, rows, value_aware=False)   # the GPU's statistics
    wmass, _ = OA.prefix_scores(q, k, None, wmp, wlp, wop, rows, value_aware=False)   # the oracle's
    assert rel_err(mass, smass) < 2e-5
    assert rel_err(mass, wmass) < 1e-4
    # the mass is the selector importance: a probability per row, mean over the G*T rows
    assert torch.allclose(mass.sum(-1).cpu().double(), torch.ones(1, 4, dtype=torch.float64), atol=1e-5)

    # read set on the GPU's mass: bit-exact with the oracle's selection of it; end to end
    # only boundary differences within the measured band
    idx = topk_ascending(mass, READ)
    assert torch.equal(idx.cpu(), OS.topk_ascending(mass.cpu(), READ))
    check_read_set("c0_read", idx.cpu(), mass.cpu(), smass, wmass, READ)

    # keep set on the same mass: 128 newest outright, the best 896 of the rest
    pos = torch.arange(n, dtype=torch.int32).view(1, 1, 1, n).expand(1, 1, 4, n).contiguous()
    keep = keep_select(pos.to(gpu), mass.view(1, 1, 4, n), KEEP, WINDOW)
    kc_cpu = keep.cpu().view(4, KEEP)
    assert torch.equal(kc_cpu, OS.keep_select(pos.view(4, n), mass.cpu().view(4, n), KEEP, WINDOW).view(4, KEEP))
    assert torch.all(kc_cpu[:, -WINDOW:] == torch.arange(n - WINDOW, n))            # the window, newest last
    assert torch.all(kc_cpu[:, 1:] > kc_cpu[:, :-1])
    # end to end: the contest part against the oracle's mass, boundary differences only
    contest = wmass.view(4, n)[:, :n - WINDOW]
    got = kc_cpu[:, :KEEP - WINDOW]
    want = OS.topk_ascending(contest, KEEP - WINDOW)
    err = rel_err(mass.cpu().view(4, n)[:, :n - WINDOW], contest)
    ok, nmis, worst = OS.boundary_mismatch_ok(got, want, contest, KEEP - WINDOW, rel=2 * err + 1e-6)
    assert ok and nmis == 0, (nmis, worst)
