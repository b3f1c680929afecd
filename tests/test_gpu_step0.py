"""GPU parity, step 0 of a sparse layer at the headline shape (
packed int4 k4v4, prefix 32768, 28/4 heads, block 32, read budget 2048): the HIP
quantizer, split-K attention, value-aware scores, read-set top-k and gather, each
checked against the CPU oracle on the same seeded inputs."""

import pytest
import torch

from maskahead_amd.kernels import gather_packed_kv, prefix_scores, splitk_attention, topk_ascending
from maskahead_amd.kernels.ops import quantize_key_groups_into, quantize_values_into
from maskahead_amd.kernels.splitk import Prefix
from maskahead_amd.workloads import CONFIGS, layer_inputs, packed_layout
from oracle import attention as OA

from _util import assert_attention_close, check_read_set, rel_err

pytestmark = pytest.mark.gpu


class _View:
    def __init__(self, p: Prefix, d: int):
        self.k_bits = self.v_bits = 4
        self.length, self.quantized_length, self.residual_length = p.n, p.nq, 0
        self.key_token_group = self.value_channel_group = 32
        self.k_q, self.k_scale, self.k_zero = p.kq, p.ks, p.kz
        self.v_q, self.v_scale, self.v_zero = p.vq, p.vs, p.vz
        self.k_fp = self.v_fp = self.k_residual = self.v_residual = None
        self.head_dim = d
        self.key_mode = "channel"


def test_config2_step0(gpu):
    sh = CONFIGS["c2"]
    q, k, v, kc, vc = layer_inputs(sh, dtype=torch.bfloat16)
    lay = packed_layout(sh.b, sh.hkv, sh.n, sh.d, device=gpu)
    kg, vg = k.to(gpu), v.to(gpu)
    quantize_key_groups_into(kg, lay["kq"], lay["ks"], lay["kz"], bits=4, token_group=32)
    quantize_values_into(vg, lay["vq"], lay["vs"], lay["vz"], bits=4, channel_group=32)
    kq, ks, kz = OA.quantize_keys(k)
    vq, vs, vz = OA.quantize_values(v)
    for name, want in (("kq", kq), ("ks", ks), ("kz", kz), ("vq", vq), ("vs", vs), ("vz", vz)):
        assert torch.equal(lay[name].cpu(), want), name            # int4 codes bit-exact

    p = Prefix(kq=lay["kq"], ks=lay["ks"], kz=lay["kz"], vq=lay["vq"], vs=lay["vs"], vz=lay["vz"],
               nq=sh.n, kb=4, vb=4)
    qg = q.to(gpu)
    out, stats = splitk_attention(qg, p, kc.to(gpu), vc.to(gpu), want_prefix=True)
    rows = torch.arange(sh.t, dtype=torch.int32)
    mass, score = prefix_scores(qg, p, stats, rows, value=True)
    idx = topk_ascending(score, sh.read_k)
    ck, cv = gather_packed_kv(_View(p, sh.d), idx)

    kd = OA.dequantize_keys(kq, ks, kz)
    vd = OA.dequantize_values(vq, vs, vz)
    wout, wmp, wlp, wop = OA.splitk_attention(q, kd, vd, kc, vc)
    assert_attention_close(out, wout)
    wmass, wscore = OA.prefix_scores(q, kd, vd.to(torch.bfloat16).float(), wmp, wlp, wop, list(range(sh.t)),
                                     value_aware=True)
    assert rel_err(mass, wmass) < 2e-5
    assert rel_err(score, wscore) < 1e-3
    # the read set: against oracle scores from the GPU's own statistics and from the
    # oracle's, each within the band its measured score error allows at the k-th value
    gmp, glp, gop = (x.cpu() for x in stats[:3])
    _, sscore = OA.prefix_scores(q, kd, vd.to(torch.bfloat16).float(), gmp, glp, gop, list(range(sh.t)),
                                 value_aware=True)
    rec = check_read_set("c2_step0", idx.cpu(), score.cpu(), sscore, wscore, sh.read_k)
    assert rec["same_stats"]["score_rel_err"] < 1e-5
    # invariants of the read set: ascending, unique, in range
    ic = idx.cpu()
    assert torch.all(ic[..., 1:] > ic[..., :-1]) and ic.min() >= 0 and ic.max() < sh.n
    # on the GPU's own indices the gather is bit-exact with the oracle's dequant
    gi = ic.unsqueeze(-1).expand(-1, -1, -1, sh.d)
    assert torch.equal(ck.cpu(), torch.gather(kd.to(torch.bfloat16), 2, gi))
    assert torch.equal(cv.cpu(), torch.gather(vd.to(torch.bfloat16), 2, gi))
