"""GPU parity, prefix scores (splitk.py:582-614): mass and value score against the CPU
oracle -- tightly when both start from the same softmax statistics, and end to end from
the oracle's own statistics."""

import pytest
import torch

from maskahead_amd.kernels.splitk import Prefix, prefix_scores, splitk_attention
from oracle import attention as OA

from _util import dequant_cpu, gpu_prefix, layer_inputs, packed_cpu, rel_err

pytestmark = pytest.mark.gpu


def _masked_rel(got, want, floor):
    got, want = got.double().cpu(), want.double().cpu()
    return float(((got - want).abs() / (want.abs() + floor)).max())


@pytest.mark.parametrize("packed", [False, True])
def test_scores_from_same_stats(gpu, packed):
    q, k, v, kc, vc = layer_inputs(hq=28, hkv=4, d=128, n=4096, t=32, seed=11, dtype=torch.bfloat16)
    if packed:
        store, nq = packed_cpu(k, v)
        p = gpu_prefix(store, nq, gpu)
        kd, vd = dequant_cpu(store, nq)
        k_used, v_dist = kd, kd.new_empty(0)
        v_dist = vd.to(torch.bfloat16).float()          # n > 256: the reference reads its bf16 copy
        v_pv = vd
    else:
        p = Prefix.dense(k.to(gpu), v.to(gpu))
        k_used, v_dist, v_pv = k.float(), v.float(), v.float()
    qg = q.to(gpu)
    out, stats = splitk_attention(qg, p, kc.to(gpu), vc.to(gpu), want_prefix=True)
    rows = [0, 3, 4, 5, 17, 30, 31]
    mass, score = prefix_scores(qg, p, stats, torch.tensor(rows, dtype=torch.int32), value=True)
    mp, lp, op = (x.cpu() for x in stats[:3])
    wmass, wscore = OA.prefix_scores(q, k_used, v_dist, mp, lp, op, rows, value_aware=True)
    assert rel_err(mass, wmass) < 2e-5
    assert rel_err(score, wscore) < 2e-5
    m_only, none = prefix_scores(qg, p, stats, torch.tensor(rows, dtype=torch.int32), value=False)
    assert none is None and torch.equal(m_only, mass)


def test_scores_end_to_end_with_mask(gpu):
    q, k, v, kc, vc = layer_inputs(hq=28, hkv=4, d=128, n=2048, t=32, seed=12, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    mask = (torch.rand((1, 4, 2048), generator=g) > 0.25).to(torch.uint8)
    p = Prefix.dense(k.to(gpu), v.to(gpu), mask=mask.to(gpu))
    qg = q.to(gpu)
    _, stats = splitk_attention(qg, p, kc.to(gpu), vc.to(gpu), want_prefix=True)
    rows = list(range(32))
    mass, score = prefix_scores(qg, p, stats, torch.arange(32, dtype=torch.int32), value=True)
    _, mp, lp, op = OA.splitk_attention(q, k, v, kc, vc, mask=mask)
    wmass, wscore = OA.prefix_scores(q, k, v, mp, lp, op, rows, mask=mask, value_aware=True)
    live = mask.bool()
    assert torch.all(mass.cpu()[~live] == 0) and torch.all(score.cpu()[~live] == 0)
    # O_p differs by bf16 rounding of p inside the PV product -> centre ~1e-4 relative
    assert rel_err(mass.cpu()[live], wmass[live]) < 2e-5
    assert rel_err(score.cpu()[live], wscore[live]) < 1e-3
