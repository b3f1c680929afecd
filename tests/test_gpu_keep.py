"""GPU parity, keep path of an eviction step: the keep set (eviction.py:325-409), the
bf16 keep score (session.py:27-40), in-place compaction (cache.py:342-367,
eviction.py:411-418) and the append of a finalized block (cache.py:423-547), each against
the CPU oracle -- and the keep score against the reference's own golden vectors."""

from pathlib import Path

import numpy as np
import pytest
import torch

from maskahead_amd.cache import PackedKVCache
from maskahead_amd.eviction import EvictionConfig, EvictionState
from maskahead_amd.kernels import gather_packed_kv
from maskahead_amd.kernels.keep import append_tokens, compact_tokens, keep_select, value_score, value_score_slots
from oracle import attention as OA
from oracle import codec as OC
from oracle import selection as OS

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden" / "golden_vectors.npz"


def _positions(rows, n, g, gap_p=0.3):
    """Strictly increasing positions with gaps, as a live set looks after evictions."""
    steps = 1 + (torch.rand((rows, n), generator=g) < gap_p).to(torch.int64) * torch.randint(1, 50, (rows, n),
                                                                                             generator=g)
    return torch.cumsum(steps, -1) - 1


@pytest.mark.parametrize("n,cap,window,sinks,pin", [
    (1, 1, 0, 0, None), (300, 40, 16, 4, None), (300, 300, 8, 0, None), (1000, 256, 128, 4, (50, 90)),
    (5000, 700, 0, 0, None), (4096, 1024, 128, 4, None), (65536, 8192, 128, 4, (1000, 1200)), (40000, 39000, 500, 0, None),
    (131072, 4096, 128, 4, (5000, 6000)), (1_050_003, 30000, 64, 4, None)])
def test_keep_select_bit_exact(gpu, n, cap, window, sinks, pin):
    g = torch.Generator().manual_seed(n + cap)
    rows = 6
    pos = _positions(rows, n, g)
    score = torch.rand((rows, n), generator=g)
    score[:, ::3] = (score[:, ::3] * 16).floor() / 16       # heavy ties
    score[:, 1::13] = 0.0
    score[:, 2::17] = -0.0
    want = OS.keep_select(pos, score, cap, window, sinks, pin)
    for dt in (torch.int32, torch.int64):
        got = keep_select(pos.to(dt).to(gpu), score.to(gpu), cap, window, sink_tokens=sinks, pin=pin)
        assert torch.equal(got.cpu(), want), dt
    # invariants: size C, ascending (= position order), the W newest present
    w = min(window, cap)
    if w:
        assert torch.all(want[:, -w:] == torch.arange(n - w, n))


def test_keep_select_per_row_pin_and_unsorted_rejected(gpu):
    g = torch.Generator().manual_seed(7)
    pos = _positions(4, 500, g)
    score = torch.rand((4, 500), generator=g)
    lo = torch.tensor([10, 20, 30, 40])
    got = keep_select(pos.to(gpu), score.to(gpu), 100, 10, pin=(lo.to(gpu), 60))
    for r in range(4):
        want = OS.keep_select(pos[r:r + 1], score[r:r + 1], 100, 10, 0, (int(lo[r]), 60))
        assert torch.equal(got[r:r + 1].cpu(), want)
    bad = pos.clone()
    bad[2, 100], bad[2, 101] = bad[2, 101], bad[2, 100]
    with pytest.raises(ValueError):
        keep_select(bad.to(gpu), score.to(gpu), 100, 10)
    # a violation exactly across a 1024-entry chunk boundary, and one inside the window
    pos2 = _positions(3, 5000, g)
    s2 = torch.rand((3, 5000), generator=g)
    pos2[1, 1024] = pos2[1, 1023]
    pos2[2, 4990] = pos2[2, 4989] - 1
    from maskahead_amd import _native as N
    from maskahead_amd.kernels.select import _state
    lib = N.load()
    st = torch.zeros((3,), dtype=torch.int32, device=gpu)
    out = torch.empty((3, 300), dtype=torch.int64, device=gpu)
    ws = torch.empty((int(lib.ma_topk_workspace_bytes(3, 5000)),), dtype=torch.uint8, device=gpu)
    state = _state(torch.device(gpu), int(lib.ma_topk_state_bytes(3)))
    pg, sg = pos2.to(gpu), s2.to(gpu)
    rc = lib.ma_keep_select(pg.data_ptr(), 1, 5000, sg.data_ptr(), 5000, 3, 5000, 300, 20, 0, None, 0, 0, 0,
                            out.data_ptr(), 300, st.data_ptr(), state.data_ptr(), state.numel(), ws.data_ptr(),
                            ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert st.cpu().tolist() == [0, 1, 1]


def _bf16(bits):
    return torch.from_numpy(bits.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("tag", ["vs_small", "vs_mid"])
def test_value_score_matches_reference_golden(gpu, tag):
    z = np.load(GOLD)
    a = torch.from_numpy(z[f"{tag}_a"])
    v = _bf16(z[f"{tag}_v"])
    want = torch.from_numpy(z[f"{tag}_score"])       # written by the reference's value_score
    got = value_score(a.to(gpu), v.to(gpu), fp32=False)
    assert torch.equal(got.cpu(), want)


@pytest.mark.parametrize("n,h", [(4096, 4), (65536, 8)])
def test_value_score_bf16_bit_exact_vs_oracle(gpu, n, h):
    g = torch.Generator().manual_seed(n)
    a = torch.softmax(torch.randn((1, h, n), generator=g) * 3, -1)
    a[..., ::11] = 0.0
    v = torch.randn((1, h, n, 128), generator=g).to(torch.bfloat16)
    # capacity-padded storage: the kernel reads a strided view
    store = torch.zeros((1, h, n + 77, 128), dtype=torch.bfloat16)
    store[:, :, :n] = v
    got = value_score(a.to(gpu), store.to(gpu)[:, :, :n], fp32=False)
    want = OA.value_score_bf16(a, v)
    assert torch.equal(got.cpu(), want)


def test_value_score_fp32_branch(gpu):
    g = torch.Generator().manual_seed(3)
    a = torch.rand((2, 3, 1000), generator=g)
    v = torch.randn((2, 3, 1000, 64), generator=g).to(torch.bfloat16)
    got = value_score(a.to(gpu), v.to(gpu), fp32=True).cpu()
    want = OA.value_score_fp32(a, v)
    assert torch.allclose(got, want, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("d,dtype,fp32", [(128, torch.bfloat16, False), (64, torch.bfloat16, False),
                                           (128, torch.float32, False), (128, torch.bfloat16, True)])
def test_value_score_slots_equals_gather_then_score(gpu, d, dtype, fp32):
    """The lookahead keep score straight from a cache's slots (ma_value_score_slots) is the
    value score of the rows gather_packed_kv returns for those slots, bit for bit: packed
    slots, 16-bit residual slots, slots outside the cache (zero rows), capacity-strided
    slot rows; and, in the bf16 branch, the oracle's value score of the oracle's dequant."""
    from _util import dequant_cpu, gpu_prefix, layer_inputs, packed_cpu

    n, tail = 640, 72
    _, k, v, _, _ = layer_inputs(hq=4, hkv=2, d=d, n=n + tail, t=4, seed=41, dtype=torch.bfloat16)
    store, nq = packed_cpu(k[:, :, :n], v[:, :, :n], pad_groups=2, pad_tokens=50)
    p = gpu_prefix(store, nq, gpu, kf=k[:, :, n:], vf=v[:, :, n:])
    g = torch.Generator().manual_seed(d)
    live, cap = 500, 530
    slots = torch.full((1, 2, cap), -7, dtype=torch.int32)
    for h in range(2):
        slots[0, h, :live] = torch.randperm(n + tail, generator=g)[:live].sort().values.to(torch.int32)
    slots[0, 1, 17] = -1                       # outside the cache: a zero row
    slots[0, 0, 33] = n + tail + 5
    a = torch.rand((1, 2, live), generator=g)
    a[..., ::9] = 0.0
    ag, sg = a.to(gpu), slots.to(gpu)
    got = value_score_slots(ag, p, sg, dtype=dtype, fp32=fp32)
    _, vg = gather_packed_kv(p, sg[..., :live].to(torch.int64), dtype=dtype)
    want = value_score(ag, vg, fp32=fp32)
    assert torch.equal(got.cpu(), want.cpu())
    if dtype == torch.bfloat16 and not fp32:
        kd, vd = dequant_cpu(store, nq)
        v_all = torch.cat([vd.to(torch.bfloat16), v[:, :, n:]], 2)
        idx = slots[..., :live].to(torch.int64)
        ok = (idx >= 0) & (idx < n + tail)
        rows = torch.gather(v_all, 2, idx.clamp(0, n + tail - 1).unsqueeze(-1).expand(-1, -1, -1, d))
        rows = torch.where(ok.unsqueeze(-1), rows, torch.zeros((), dtype=rows.dtype))
        assert torch.equal(got.cpu(), OA.value_score_bf16(a, rows))


@pytest.mark.parametrize("kind", ["survivors", "arbitrary"])
def test_compact_in_place(gpu, kind):
    g = torch.Generator().manual_seed(11)
    b, h, n, cap_extra, d, c = 1, 8, 6000, 300, 128, 900
    k = torch.randn((b, h, n + cap_extra, d), generator=g).to(torch.bfloat16)
    v = torch.randn((b, h, n + cap_extra, d), generator=g).to(torch.bfloat16)
    if kind == "survivors":
        pos = _positions(b * h, n, g)
        keep = OS.keep_select(pos, torch.rand((b * h, n), generator=g), c, 128, 4).view(b, h, c)
    else:   # any gather: permuted, repeated and out-of-range indices
        keep = torch.randint(-5, n + 5, (b, h, c), generator=g)
    kg, vg = k.to(gpu), v.to(gpu)
    compact_tokens([kg, vg], keep.to(gpu), n)
    kc = keep.clamp(0, n - 1)
    valid = ((keep >= 0) & (keep < n)).unsqueeze(-1)
    for got, src in ((kg, k), (vg, v)):
        want = torch.from_numpy(OC.compact_rows(src[:, :, :n].view(torch.int16).numpy(), kc.numpy())).view(torch.bfloat16)
        want = torch.where(valid, want, torch.zeros_like(want))
        assert torch.equal(got[:, :, :c].cpu(), want)
        assert torch.equal(got[:, :, n:].cpu(), src[:, :, n:])   # rows past the live range untouched


def test_eviction_state_survivors_and_compact(gpu):
    g = torch.Generator().manual_seed(5)
    L, B, H, n = 2, 1, 4, 3000
    st = EvictionState(num_layers=L, batch_size=B, num_kv_heads=H, capacity=64, device=gpu)
    pos = _positions(1, n, g)[0]
    st.append(pos.to(gpu))
    for l in range(L):
        for _ in range(3):
            st.observe(l, torch.rand((B, H, n), generator=g).to(gpu), 0.9)
    cfg = EvictionConfig(policy="lookahead", recent_window=64, capacity_floor=256, sink_tokens=4)
    score = torch.rand((L, B, H, n), generator=g)
    keep = st.survivors(cfg, 500, None, score.to(gpu))
    want = OS.keep_select(pos.expand(L, B, H, n), score, 500, 64, 4)
    assert torch.equal(keep.cpu(), want)
    # ema_recent: ranks on the bias-corrected EMA
    cfg2 = EvictionConfig(policy="ema_recent", recent_window=32, capacity_floor=256)
    ghat = torch.stack([st.corrected(l, 0.9) for l in range(L)]).cpu()
    keep2 = st.survivors(cfg2, 400)
    assert torch.equal(keep2.cpu(), OS.keep_select(pos.expand(L, B, H, n), ghat, 400, 32))
    # recent: the C newest, sinks first
    keep3 = st.survivors(EvictionConfig(policy="recent", sink_tokens=2), 300)
    assert torch.equal(keep3.cpu(), OS.keep_select(pos.expand(L, B, H, n), pos.expand(L, B, H, n).float(), 300, 0, 2))
    before = {name: getattr(st, name)[..., :n].cpu().clone() for name in ("g", "n", "pos", "phys")}
    st.compact(keep)
    assert st.live == 500
    for name, old in before.items():
        assert torch.equal(getattr(st, name)[..., :500].cpu(), old.gather(-1, want)), name


def test_append_tokens(gpu):
    g = torch.Generator().manual_seed(2)
    dst = torch.zeros((2, 3, 104, 128), dtype=torch.bfloat16)
    src = torch.randn((2, 3, 32, 128), generator=g)
    dg = dst.to(gpu)
    append_tokens(src.to(gpu), dg, 40)                       # f32 -> bf16, round to nearest even
    append_tokens(src.to(torch.bfloat16).to(gpu), dg, 72)   # bf16 copy
    want = dst.clone()
    want[:, :, 40:72] = src.to(torch.bfloat16)
    want[:, :, 72:104] = src.to(torch.bfloat16)
    assert torch.equal(dg.cpu(), want)
    with pytest.raises(ValueError):
        append_tokens(src.to(gpu), dg, 80)                  # past the capacity


@pytest.mark.parametrize("residual_tokens", [0, 32, 64])
def test_fused_packed_append_equals_quantizer_path(gpu, residual_tokens):
    """PackedKVCache.stage_layer through ma_append_packed (one call: quantize from
    [residual | new] directly, then the residual shifted down in place) writes the same
    bytes as the path that builds [residual | new] and calls the quantizers and the append
    kernel (the reference's stage_layer, cache.py:423-548), over appends that hit every
    case: new tokens only appended to the residual, whole groups quantized with the kept
    residual moving down over rows it is read from, and a long prefill.  The quantizer path
    itself is pinned against the oracle and the reference's golden vectors."""
    from maskahead_amd.config import QuantizationConfig

    g = torch.Generator().manual_seed(71)
    L, B, H, D = 2, 2, 3, 128
    quant = QuantizationConfig(residual_tokens=residual_tokens)
    caches = [PackedKVCache(num_layers=L, batch_size=B, num_kv_heads=H, head_dim=D, max_tokens=4096, quant=quant,
                            device=gpu) for _ in range(2)]
    caches[1]._append_fused = lambda key, value: False        # the quantizer path
    names = ("k_q", "k_scale", "k_zero", "v_q", "v_scale", "v_zero", "k_residual", "v_residual")
    seen = set()
    for n in (300, 32, 32, 7, 32, 32, 25, 32, 64, 32):
        kv = [(torch.randn((B, H, n, D), generator=g) * 3).to(torch.bfloat16) for _ in range(2 * L)]
        for c in caches:
            plan = c.begin_append(n)
            for layer in range(L):
                c.stage_layer(layer, kv[2 * layer].to(gpu), kv[2 * layer + 1].to(gpu))
            c.commit_append()
        seen.add((plan.quantize_from_residual > 0, plan.quantize_from_residual < plan.old_residual,
                  plan.new_residual > 0))
        a, b = caches
        assert (a.length, a.quantized_length, a.residual_length) == (b.length, b.quantized_length, b.residual_length)
        ql, rl = a.quantized_length, a.residual_length
        for name in names:
            x, y = getattr(a, name), getattr(b, name)
            cut = ql // 32 if name.startswith("k_") and "residual" not in name else ql if "residual" not in name \
                else rl
            assert torch.equal(x[:, :, :, :cut].cpu(), y[:, :, :, :cut].cpu()), (n, name)
    if residual_tokens:
        # the in-place shift over its own source rows and the append-only case both ran
        assert (True, True, True) in seen and (False, True, True) in seen
