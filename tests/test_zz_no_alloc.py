"""GPU parity of ma_splitk_attention_noalloc, the split-K attention entry point that keeps
its split partials in a library-owned device array instead of a caller workspace (for
callers that cannot allocate).  It runs the same kernels with the same split plan as
ma_splitk_attention, so its outputs must be bit-identical; checked on two calls in a row,
the second smaller than the first, so the second reuses the array the first left dirty."""

import ctypes

import pytest
import torch

from maskahead_amd import _native as N
from maskahead_amd.kernels.splitk import Prefix

from _util import gpu_prefix, layer_inputs, packed_cpu, same_bits

pytestmark = pytest.mark.gpu


def _call(name, q, pre, kc, vc, *, with_stats, workspace=None):
    """One call of `name` through the C ABI; returns (out, mp, lp, op)."""
    lib = N.load()
    b, hq, t, d = q.shape
    hkv = kc.shape[1]
    r = (hq // hkv) * t
    out = torch.empty_like(q)
    mp = lp = op = None
    if with_stats:
        mp = torch.empty((b, hkv, r), device=q.device, dtype=torch.float32)
        lp = torch.empty_like(mp)
        op = torch.empty((b, hkv, r, d), device=q.device, dtype=q.dtype)
    args = [N.t4(q), b, hq, t, d, ctypes.byref(pre.native()), hkv, N.t4(kc), N.t4(vc), kc.shape[2], 0, 0, 0,
            d ** -0.5, N.t4(out), N.ptr(mp), N.ptr(lp), N.ptr(op), 0]
    if workspace is not None:
        args += [workspace.data_ptr(), workspace.numel()]
    args.append(N.stream_of(q))
    N.check(getattr(lib, name)(*args), name)
    return out, mp, lp, op


def _both(q, pre, kc, vc, with_stats):
    lib = N.load()
    b, hq, t, d = q.shape
    hkv = kc.shape[1]
    ws_bytes = int(lib.ma_splitk_workspace_bytes(b, hkv, hq, t, d, pre.nq, pre.nf, 0))
    assert 0 < ws_bytes <= int(lib.ma_splitk_noalloc_max_bytes())
    ws = torch.empty((ws_bytes,), device=q.device, dtype=torch.uint8)
    want = _call("ma_splitk_attention", q, pre, kc, vc, with_stats=with_stats, workspace=ws)
    got = _call("ma_splitk_attention_noalloc", q, pre, kc, vc, with_stats=with_stats)
    torch.cuda.synchronize()
    return got, want


def test_noalloc_matches_workspace_entry_point_twice(gpu):
    # call 1: config-2 shape, packed int4 prefix of 32 768 tokens, with prefix statistics
    q, k, v, kc, vc = layer_inputs(hq=28, hkv=4, d=128, n=32768, t=32, seed=1234, dtype=torch.bfloat16)
    store, nq = packed_cpu(k, v)
    pre = gpu_prefix(store, nq, gpu)
    got, want = _both(q.to(gpu), pre, kc.to(gpu), vc.to(gpu), with_stats=True)
    for g, w in zip(got, want):
        assert same_bits(g, w)
    # call 2, smaller: a bf16 prefix of 1 000 tokens with dead slots, fewer heads, no stats
    q2, k2, v2, kc2, vc2 = layer_inputs(hq=8, hkv=2, d=128, n=1000, t=16, seed=7, dtype=torch.bfloat16)
    mask = (torch.rand((1, 2, 1000), generator=torch.Generator().manual_seed(8)) > 0.25).to(torch.uint8)
    pre2 = Prefix.dense(k2.to(gpu), v2.to(gpu), mask=mask.to(gpu))
    got2, want2 = _both(q2.to(gpu), pre2, kc2.to(gpu), vc2.to(gpu), with_stats=False)
    assert same_bits(got2[0], want2[0])
    assert torch.isfinite(got2[0].float()).all()


def test_noalloc_rejects_calls_beyond_its_array(gpu):
    # 1 024 rows per KV head over 64 KV heads needs more partials than the fixed array holds;
    # the size check runs on the host before any launch
    lib = N.load()
    need = int(lib.ma_splitk_workspace_bytes(8, 8, 32, 256, 128, 0, 64, 0))
    assert need > int(lib.ma_splitk_noalloc_max_bytes())
    q = torch.zeros((8, 32, 256, 128), device=gpu, dtype=torch.bfloat16)
    kv = torch.zeros((8, 8, 64, 128), device=gpu, dtype=torch.bfloat16)
    kc = torch.zeros((8, 8, 256, 128), device=gpu, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="scratch"):
        _call("ma_splitk_attention_noalloc", q, Prefix.dense(kv, kv), kc, kc, with_stats=False)
