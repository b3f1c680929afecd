"""GPU parity of the GQA-reduced VALU score pass (prefix_scores with at most 16 selection
rows per KV head, forced: the default path takes the MFMA pass, which measured as fast;
reference splitk.py:321-371, 582-614): mass and value score against the CPU oracle from
the same softmax statistics, and against the MFMA pass forced on the same call, for G 7 and G 4 with T2 in {1, 2} (and 4), packed and 16-bit prefixes, dead slots,
a partial last unit, an f32 prefix and a device row table."""

import pytest
import torch

from maskahead_amd import _native as N
from maskahead_amd.kernels.splitk import Prefix, prefix_scores, splitk_attention
from oracle import attention as OA

from _util import dequant_cpu, gpu_prefix, layer_inputs, packed_cpu, rel_err

pytestmark = pytest.mark.gpu

AUTO, MFMA, VALU = 0, 1, 2


def _scores(lib, mode, qg, p, stats, rows, value):
    prev = lib.ma_prefix_scores_path(mode)
    try:
        return prefix_scores(qg, p, stats, rows, value=value)
    finally:
        lib.ma_prefix_scores_path(prev)


def _case(gpu, hq, packed, n, seed, tail=0, dead=0.0):
    q, k, v, kc, vc = layer_inputs(hq=hq, hkv=4, d=128, n=n + tail, t=32, seed=seed, dtype=torch.bfloat16)
    mask = None
    if dead:
        mask = (torch.rand((1, 4, n + tail), generator=torch.Generator().manual_seed(seed + 1)) >= dead)
        mask = mask.to(torch.uint8)
    if packed:
        store, nq = packed_cpu(k[:, :, :n], v[:, :, :n], pad_groups=1, pad_tokens=32)
        kf = k[:, :, n:] if tail else None
        vf = v[:, :, n:] if tail else None
        p = gpu_prefix(store, nq, gpu, kf=kf, vf=vf, mask=mask)
        kd, vd = dequant_cpu(store, nq)
        if tail:
            kd = torch.cat([kd, k[:, :, n:].float()], 2)
            vd = torch.cat([vd, v[:, :, n:].float()], 2)
        k_used, v_dist = kd, vd.to(torch.bfloat16).float()     # n > 256: the reference reads its bf16 copy
    else:
        p = Prefix.dense(k.to(gpu), v.to(gpu), mask=None if mask is None else mask.to(gpu))
        k_used, v_dist = k.float(), v.float()
    qg = q.to(gpu)
    _, stats = splitk_attention(qg, p, kc.to(gpu), vc.to(gpu), want_prefix=True)
    return q, qg, p, stats, k_used, v_dist, mask


@pytest.mark.parametrize("hq,rows", [(28, [31]), (28, [4, 31]), (16, [0]), (16, [7, 19]), (16, [1, 2, 30, 31])])
@pytest.mark.parametrize("packed", [False, True])
def test_valu_scores_against_oracle(gpu, hq, rows, packed):
    lib = N.load()
    n, tail = (4064, 40) if packed else (2500, 0)
    q, qg, p, stats, k_used, v_dist, mask = _case(gpu, hq, packed, n, seed=81 + hq + len(rows), tail=tail,
                                                  dead=0.1)
    rt = torch.tensor(rows, dtype=torch.int32)
    mass, score = _scores(lib, VALU, qg, p, stats, rt, True)
    mp, lp, op = (x.cpu() for x in stats[:3])
    wmass, wscore = OA.prefix_scores(q, k_used, v_dist, mp, lp, op, rows, mask=mask, value_aware=True)
    live = torch.ones_like(wmass, dtype=torch.bool) if mask is None else mask.bool()
    assert torch.all(mass.cpu()[~live] == 0) and torch.all(score.cpu()[~live] == 0)
    assert rel_err(mass.cpu()[live], wmass[live]) < 2e-5
    assert rel_err(score.cpu()[live], wscore[live]) < 2e-5
    # the padded MFMA pass on the same call: the same sums in another order; auto takes it
    fmass, fscore = _scores(lib, MFMA, qg, p, stats, rt, True)
    amass, ascore = _scores(lib, AUTO, qg, p, stats, rt, True)
    assert torch.equal(fmass, amass) and torch.equal(fscore, ascore)
    assert rel_err(mass.cpu()[live], fmass.cpu()[live]) < 1e-5
    assert rel_err(score.cpu()[live], fscore.cpu()[live]) < 1e-5
    # mass only, rows from a device table
    m_only, none = _scores(lib, VALU, qg, p, stats, rt.to(gpu), False)
    assert none is None and torch.equal(m_only, mass)


def test_valu_scores_f32_prefix(gpu):
    """An f32 prefix (element-wise staging): K enters the dot as bf16, V the distance as f32."""
    lib = N.load()
    q, k, v, kc, vc = layer_inputs(hq=28, hkv=4, d=128, n=1000, t=32, seed=95, dtype=torch.float32)
    p = Prefix.dense(k.to(gpu), v.to(gpu))
    qg = q.to(gpu)
    _, stats = splitk_attention(qg, p, kc.to(gpu), vc.to(gpu), want_prefix=True)
    rows = [2, 29]
    mass, score = _scores(lib, VALU, qg, p, stats, torch.tensor(rows, dtype=torch.int32), True)
    mp, lp, op = (x.cpu() for x in stats[:3])
    wmass, wscore = OA.prefix_scores(q, k, v, mp, lp, op, rows, value_aware=True)   # q, K rounded to bf16 inside
    assert rel_err(mass, wmass) < 2e-5
    assert rel_err(score, wscore) < 2e-5


def test_valu_path_limits(gpu):
    """The VALU pass takes at most 16 selection rows: forced beyond, the call fails; auto
    sends every row count (here 21) to the MFMA pass."""
    lib = N.load()
    q, qg, p, stats, k_used, v_dist, _ = _case(gpu, 28, True, 1024, seed=90)
    rows = torch.tensor([0, 1, 2], dtype=torch.int32)          # 7 * 3 = 21 rows
    with pytest.raises(N.KernelUnavailableError):
        _scores(lib, VALU, qg, p, stats, rows, False)
    mass, _ = _scores(lib, AUTO, qg, p, stats, rows, False)
    fmass, _ = _scores(lib, MFMA, qg, p, stats, rows, False)
    assert torch.equal(mass, fmass)
    assert lib.ma_prefix_scores_path(3) == -1
