"""GPU: lane bases beyond 31 bits.  The split-K and score kernels compute a (batch, KV
head) lane's base pointers with 32-bit products when every lane offset of the prefix fits
in 31 bits and with 64-bit ones otherwise.  Here batch 1 of the packed keys lies 2 GiB past
batch 0 (its lane offsets exceed 2^31 bytes, so the 64-bit path runs); the attention
output, the prefix statistics, the scores and the read set of the fused score + select
(whose first histogram level the 64-bit score kernel leaves to the select's own launch)
must be bit-identical to those of the same prefix stored compactly (the 32-bit path)."""

import pytest
import torch

from maskahead_amd.kernels import prefix_scores_topk
from maskahead_amd.kernels.splitk import Prefix, prefix_scores, splitk_attention

from _util import gpu_prefix, layer_inputs, packed_cpu

pytestmark = pytest.mark.gpu

_GIB2 = 1 << 31


def test_lane_offsets_beyond_31_bits(gpu):
    b, hq, hkv, d, n, t = 2, 8, 2, 128, 2048, 16
    q, k, v, kc, vc = layer_inputs(b=b, hq=hq, hkv=hkv, d=d, n=n, t=t, seed=41, dtype=torch.bfloat16)
    store, nq = packed_cpu(k, v)
    compact = gpu_prefix(store, nq, gpu)
    # the same key codes with batch 1 placed 2 GiB after batch 0
    kq = store["kq"]
    per_batch = kq[0].numel()
    big = torch.zeros((_GIB2 + per_batch,), dtype=torch.uint8, device=gpu)
    far = big.as_strided(kq.shape, (_GIB2,) + tuple(kq.stride()[1:]))
    far.copy_(kq.to(gpu))
    assert far.stride(0) * (b - 1) > (1 << 31) - 1
    wide = Prefix(kq=far, ks=compact.ks, kz=compact.kz, vq=compact.vq, vs=compact.vs, vz=compact.vz,
                  nq=nq, kb=4, vb=4, kg=32, vg=32)
    qg, kcg, vcg = q.to(gpu), kc.to(gpu), vc.to(gpu)
    out_c, st_c = splitk_attention(qg, compact, kcg, vcg, want_prefix=True)
    out_w, st_w = splitk_attention(qg, wide, kcg, vcg, want_prefix=True)
    assert torch.equal(out_c, out_w)
    for x, y in zip(st_c[:3], st_w[:3]):
        assert torch.equal(x, y)
    rows = list(range(t))
    m_c, s_c = prefix_scores(qg, compact, st_c, rows, value=True)
    m_w, s_w = prefix_scores(qg, wide, st_w, rows, value=True)
    assert torch.equal(m_c, m_w)
    assert torch.equal(s_c, s_w)
    fm_c, fs_c, idx_c = prefix_scores_topk(qg, compact, st_c, rows, 300, value=True)
    fm_w, fs_w, idx_w = prefix_scores_topk(qg, wide, st_w, rows, 300, value=True)
    assert torch.equal(fs_c, s_c) and torch.equal(fs_w, s_w)
    assert torch.equal(idx_c, idx_w)
    assert torch.equal(idx_c, torch.topk(s_c, 300).indices.sort(-1).values)
    del big, far
