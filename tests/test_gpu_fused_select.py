"""GPU: the score pass with the read-set top-k's first histogram level built in-kernel
(ma_prefix_scores_hist + ma_topk_select_hist_ready, select.prefix_scores_topk) returns
exactly what prefix_scores followed by topk_ascending returns (session.py:1418-1438):
identical mass and score bits and identical indices, for packed and 16-bit prefixes,
masked and unmasked, mass and score ranks, the GQA-reduced VALU pass (whose histogram
comes from the select's own level-0 launch), mass passes over more rows than one launch
takes, and workgroups that count their keys in several blocks.  Each call must leave the
shared select state zero."""

import pytest
import torch

from maskahead_amd.kernels import select as SE
from maskahead_amd.kernels.splitk import Prefix, prefix_scores, splitk_attention
from maskahead_amd.kernels import prefix_scores_topk, topk_ascending

from _util import gpu_prefix, layer_inputs, packed_cpu

pytestmark = pytest.mark.gpu


def _state_is_zero(gpu) -> bool:
    key = (gpu.index if gpu.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(gpu).cuda_stream)
    st = SE._STATES.get(key)
    return st is None or int(st.count_nonzero()) == 0


def _compare(gpu, q, p, kc, vc, rows, k, value, rank):
    qg = q.to(gpu)
    _, stats = splitk_attention(qg, p, kc.to(gpu), vc.to(gpu), want_prefix=True)
    used = stats[3]
    mass, score = prefix_scores(qg, p, stats, rows, value=value)
    want_idx = topk_ascending(score if rank == "score" else mass, k, used.mask)
    fm, fs, fidx = prefix_scores_topk(qg, p, stats, rows, k, value=value, rank=rank)
    assert torch.equal(fm, mass)
    if value:
        assert torch.equal(fs, score)
    assert torch.equal(fidx, want_idx)
    assert _state_is_zero(gpu)
    return fidx


@pytest.mark.parametrize("dead", [0.0, 0.2])
@pytest.mark.parametrize("rank", ["score", "mass"])
def test_fused_packed(gpu, dead, rank):
    q, k, v, kc, vc = layer_inputs(hq=28, hkv=4, d=128, n=8192 + 40, t=32, seed=21, dtype=torch.bfloat16)
    n = 8192
    mask = None
    if dead:
        mask = (torch.rand((1, 4, n + 40), generator=torch.Generator().manual_seed(3)) >= dead).to(torch.uint8)
    store, nq = packed_cpu(k[:, :, :n], v[:, :, :n], pad_groups=1, pad_tokens=32)
    p = gpu_prefix(store, nq, gpu, kf=k[:, :, n:], vf=v[:, :, n:], mask=mask)
    _compare(gpu, q, p, kc, vc, list(range(32)), 1024, value=rank == "score", rank=rank)


def test_fused_dense_row_table(gpu):
    """A bf16 prefix and selection rows out of order (row tables)."""
    q, k, v, kc, vc = layer_inputs(hq=28, hkv=4, d=128, n=3000, t=32, seed=22, dtype=torch.bfloat16)
    p = Prefix.dense(k.to(gpu), v.to(gpu))
    rows = torch.tensor([3, 17, 5, 30, 8, 9], dtype=torch.int32)
    _compare(gpu, q, p, kc, vc, rows, 700, value=True, rank="score")


def test_fused_small_row_pass(gpu):
    """One selection position (7 rows per KV head): the GQA-reduced VALU pass, whose level-0
    histogram comes from the select's own histogram kernel."""
    q, k, v, kc, vc = layer_inputs(hq=28, hkv=4, d=128, n=4096, t=32, seed=23, dtype=torch.bfloat16)
    store, nq = packed_cpu(k, v)
    p = gpu_prefix(store, nq, gpu)
    _compare(gpu, q, p, kc, vc, [31], 512, value=True, rank="score")


def test_fused_mass_passes(gpu):
    """672 selection rows (96 positions x G 7): mass-only passes of at most 512 rows, the
    histogram from the last pass's final mass."""
    q, k, v, kc, vc = layer_inputs(hq=28, hkv=4, d=128, n=4096, t=96, seed=24, dtype=torch.bfloat16)
    store, nq = packed_cpu(k, v)
    p = gpu_prefix(store, nq, gpu)
    _compare(gpu, q, p, kc, vc, list(range(96)), 300, value=False, rank="mass")


def test_fused_key_blocks(gpu):
    """A lane long enough that every workgroup runs more than 64 tiles, so its keys are
    counted in several blocks during the tile loop (one KV head, 1.1 M entries)."""
    n = 1_100_000 // 64 * 64
    g = torch.Generator().manual_seed(25)
    q = torch.randn((1, 4, 32, 128), generator=g).to(torch.bfloat16)
    k = torch.randn((1, 1, n, 128), generator=g).to(torch.bfloat16)
    v = torch.randn((1, 1, n, 128), generator=g).to(torch.bfloat16)
    kc = torch.randn((1, 1, 32, 128), generator=g).to(torch.bfloat16)
    p = Prefix.dense(k.to(gpu), v.to(gpu))
    _compare(gpu, q, p, kc, kc, list(range(32)), 50_000, value=True, rank="score")


def test_fused_repeated_calls(gpu):
    """Back-to-back fused calls of different shapes share the select state; each leaves it
    zero, so the plain select after them is still exact."""
    for seed, n, kk in ((31, 5000, 123), (32, 9000, 4000), (33, 2048, 2048)):
        q, k, v, kc, vc = layer_inputs(hq=16, hkv=4, d=128, n=n, t=8, seed=seed, dtype=torch.bfloat16)
        p = Prefix.dense(k.to(gpu), v.to(gpu))
        _compare(gpu, q, p, kc, vc, list(range(8)), kk, value=True, rank="score")
