"""Packed eviction rebuild on the GPU (ma_rebuild_plan + ma_rebuild_packed) against the
reference's own vectors and the CPU oracle (oracle/rebuild.py): every written byte of the
new storage, the lengths and the eviction state's new slots, bit-exact."""

from __future__ import annotations

import pytest
import torch

from maskahead_amd.cache import PackedKVCache
from maskahead_amd.config import QuantizationConfig
from maskahead_amd.eviction import EvictionConfig, EvictionState
from maskahead_amd.kernels.rebuild import rebuild_plan
from maskahead_amd.runtime.session import evict_to
from oracle import attention as OA
from oracle import rebuild as OR
from tests._util import REBUILD_CASES, rebuild_case, same_bits

pytestmark = pytest.mark.gpu

NAMES = (("kq", "k_q"), ("ks", "k_scale"), ("kz", "k_zero"), ("vq", "v_q"), ("vs", "v_scale"), ("vz", "v_zero"),
         ("kr", "k_residual"), ("vr", "v_residual"))


def _cache_from(store: dict, lens: tuple, dev, *, stage: bool = False, residual_tokens: int = 32) -> PackedKVCache:
    """A GPU cache holding `store` (oracle layout) with the given lengths; storage padded
    past the written part so strides are capacity strides, as in a live cache."""
    L, B, H = store["kq"].shape[:3]
    D = store["kq"].shape[4]
    cache = PackedKVCache(num_layers=L, batch_size=B, num_kv_heads=H, head_dim=D, max_tokens=1 << 20,
                          quant=QuantizationConfig(residual_tokens=residual_tokens), device=dev)
    length, ql, rl, dropped = lens
    for short, name in NAMES:
        src = store[short]
        shape = list(src.shape)
        shape[3] += 37 if short in ("kr", "vr") else (3 if short in ("kq", "ks", "kz") else 96)
        t = torch.full(shape, 0x55 if src.dtype == torch.uint8 else 7.0, dtype=src.dtype)
        t[:, :, :, :src.shape[3]] = src
        setattr(cache, name, t.to(dev))
    cache.length, cache.quantized_length, cache.residual_length, cache.dropped = lens
    cache.stage = stage
    return cache


def _state_from(pos: torch.Tensor, phys: torch.Tensor, dev) -> EvictionState:
    L, B, H, live = pos.shape
    st = EvictionState(num_layers=L, batch_size=B, num_kv_heads=H, capacity=live + 5, device=dev)
    st.pos[..., :live] = pos.to(st.pos_dtype).to(dev)
    st.phys[..., :live] = phys.to(torch.int32).to(dev)
    st.live = live
    return st


def _check_cache(cache: PackedKVCache, want: dict, want_lens: tuple):
    assert (cache.length, cache.quantized_length, cache.residual_length, cache.dropped) == want_lens
    ng, ql, rl = want_lens[1] // 32, want_lens[1], want_lens[2]
    cut = {"kq": ng, "ks": ng, "kz": ng, "vq": ql, "vs": ql, "vz": ql, "kr": rl, "vr": rl}
    for short, name in NAMES:
        got = getattr(cache, name)[:, :, :, :cut[short]]
        assert same_bits(got, want[short]), short


@pytest.mark.parametrize("tag", REBUILD_CASES)
def test_evict_matches_reference_vectors(gpu, tag):
    """The reference's _evict_to on a seeded cache (lazy, a second lazy eviction of a
    rebuilt cache, full, staged bf16 + unadmitted tail, whole-group tail)."""
    c = rebuild_case(tag)
    cache = _cache_from(c["in"], c["in_lens"], gpu, stage=c["stage_mode"])
    st = _state_from(c["pos"], c["phys"], gpu)
    cfg = EvictionConfig(policy="recent", recent_window=c["recent_window"], capacity_floor=max(1, c["recent_window"]),
                         compaction=c["mode"], repack_below=c["repack_below"])
    evict_to(cache, st, c["keep"].to(gpu), cfg, next_position=c["next_position"])
    torch.cuda.synchronize()
    _check_cache(cache, c["out"], c["out_lens"])
    assert torch.equal(st.phys[..., :st.live].cpu().to(torch.int64), c["out_phys"])


def _random_cache(seed: int, *, L: int, H: int, D: int, n_q: int, n_r: int):
    """Oracle-quantized storage of n_q tokens + an n_r-token bf16 residual."""
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn((L, 1, H, n_q, D), generator=g) *
         torch.empty((L, 1, H, 1, D)).log_normal_(0, 0.5, generator=g)).to(torch.bfloat16)
    v = torch.randn((L, 1, H, n_q, D), generator=g).to(torch.bfloat16)
    kq, ks, kz = OA.quantize_keys(k.reshape(L, H, n_q, D))
    vq, vs, vz = OA.quantize_values(v.reshape(L, H, n_q, D))
    store = {"kq": kq, "ks": ks, "kz": kz, "vq": vq, "vs": vs, "vz": vz}
    store = {x: t.reshape(L, 1, H, *t.shape[2:]) for x, t in store.items()}
    store["kr"] = torch.randn((L, 1, H, n_r, D), generator=g).to(torch.bfloat16)
    store["vr"] = torch.randn((L, 1, H, n_r, D), generator=g).to(torch.bfloat16)
    return store, (n_q + n_r, n_q, n_r, 0), g


def _clustered_keep(g, L, H, n, C, window):
    """Keep sets in position order: the window, some dense key groups, random others."""
    score = torch.rand((L, 1, H, n), generator=g)
    grp = torch.arange(n) // 32
    for lane in range(L * H):
        dense = torch.randperm(n // 32, generator=g)[: 1 + lane % 5]
        score[lane // H, 0, lane % H] += 2.0 * torch.isin(grp, dense)
    score[..., n - window:] = 1e9
    keep = score.topk(C, dim=-1).indices
    return keep.sort(dim=-1).values


@pytest.mark.parametrize("mode,repack,seed", [("lazy", 0.5, 11), ("lazy", 1.0, 12), ("full", 1.0, 13)])
def test_evict_random_vs_oracle(gpu, mode, repack, seed):
    """head_dim 128, 8 lanes, 2048 quantized + 96 residual tokens, 640 survivors."""
    L, H, D, n_q, n_r, C, W = 2, 4, 128, 2048, 96, 640, 48
    store, lens, g = _random_cache(seed, L=L, H=H, D=D, n_q=n_q, n_r=n_r)
    n = lens[0]
    pos = torch.arange(n).expand(L, 1, H, n).clone()
    phys = pos.clone()
    keep = _clustered_keep(g, L, H, n, C, W)
    want, want_lens, want_phys = OR.evict(store, lens, pos, phys, keep, next_position=n, stage_mode=False,
                                          mode=mode, repack_below=repack, recent_window=W)
    cache = _cache_from(store, lens, gpu)
    st = _state_from(pos, phys, gpu)
    cfg = EvictionConfig(policy="recent", recent_window=W, capacity_floor=W, compaction=mode, repack_below=repack)
    evict_to(cache, st, keep.to(gpu), cfg, next_position=n)
    torch.cuda.synchronize()
    _check_cache(cache, want, want_lens)
    assert torch.equal(st.phys[..., :C].cpu().to(torch.int64), want_phys)


def test_evict_long_prefix_vs_oracle(gpu):
    """32 768 quantized tokens per lane (the benchmark's prefix), 4 lanes, keep 4096."""
    L, H, D, n_q, n_r, C, W = 1, 4, 128, 32768, 32, 4096, 128
    store, lens, g = _random_cache(21, L=L, H=H, D=D, n_q=n_q, n_r=n_r)
    n = lens[0]
    pos = torch.arange(n).expand(L, 1, H, n).clone()
    keep = _clustered_keep(g, L, H, n, C, W)
    want, want_lens, want_phys = OR.evict(store, lens, pos, pos, keep, next_position=n, stage_mode=False,
                                          mode="lazy", repack_below=0.5, recent_window=W)
    cache = _cache_from(store, lens, gpu)
    st = _state_from(pos, pos, gpu)
    cfg = EvictionConfig(policy="recent", recent_window=W, capacity_floor=W, compaction="lazy", repack_below=0.5)
    evict_to(cache, st, keep.to(gpu), cfg, next_position=n)
    torch.cuda.synchronize()
    _check_cache(cache, want, want_lens)
    assert torch.equal(st.phys[..., :C].cpu().to(torch.int64), want_phys)


@pytest.mark.parametrize("live", [300, 5000])
def test_plan_out_of_order_lanes(gpu, live):
    """Lanes whose live entries are not in (position, slot) order: the plan sorts them in
    LDS and still returns the reference's lists (oracle.plan sorts with torch)."""
    L, H, n_q = 2, 2, 8192
    g = torch.Generator().manual_seed(live)
    pos = torch.stack([torch.randperm(20000, generator=g)[:live] for _ in range(L * H)]).view(L, 1, H, live)
    phys = torch.stack([torch.randperm(n_q + 64, generator=g)[:live] for _ in range(L * H)]).view(L, 1, H, live)
    lens = (n_q + 64, n_q, 64, 0)
    want = OR.plan(phys, pos, lens, tail=0, stage_mode=False, mode="lazy", repack_below=0.25, recent_window=40)
    st = _state_from(pos, phys, gpu)
    got = rebuild_plan(st.phys, st.pos, live, quantized_length=n_q, need=8, tail_groups=0, window=40)
    for a, b in zip(got, (want[0], want[1], want[3])):
        assert torch.equal(a.cpu(), b)


def test_rebuild_direct_lists_and_errors(gpu):
    """cache.rebuild with hand-made lists: padding (-1) copies group 0 / writes zeros, the
    remap names every moved slot; a list entry outside the cache raises."""
    store, lens, g = _random_cache(5, L=1, H=2, D=64, n_q=128, n_r=16)
    gb = torch.tensor([[2, -1], [0, 3]]).view(1, 1, 2, 2)
    enc = torch.tensor([[5, 130, -1], [140, 7, 9]]).view(1, 1, 2, 3)
    ga = torch.empty((1, 1, 2, 0), dtype=torch.int64)
    stg = torch.tensor([[131, -1], [129, 100]]).view(1, 1, 2, 2)
    want, want_lens, want_remap = OR.rebuild(store, lens, gb, enc, ga, stg)
    cache = _cache_from(store, lens, gpu)
    remap = cache.rebuild(gb.to(gpu), enc.to(gpu), ga.to(gpu), stg.to(gpu))
    torch.cuda.synchronize()
    _check_cache(cache, want, want_lens)
    assert torch.equal(remap.cpu(), want_remap)
    cache = _cache_from(store, lens, gpu)
    with pytest.raises(RuntimeError):
        cache.rebuild(gb.to(gpu), torch.tensor([[5, 144, -1], [1, 2, 3]]).view(1, 1, 2, 3).to(gpu), ga.to(gpu),
                      stg.to(gpu))
    # check=False: the same error, raised by the next check instead of the call
    cache = _cache_from(store, lens, gpu)
    cache._rebuild(gb.to(gpu), torch.tensor([[5, 144, -1], [1, 2, 3]]).view(1, 1, 2, 3).to(gpu), ga.to(gpu),
                   stg.to(gpu), check=False)
    with pytest.raises(RuntimeError):
        cache.check_rebuild()
    cache.check_rebuild()                         # raised once, then nothing pending
    cache = _cache_from(store, lens, gpu)
    cache._rebuild(gb.to(gpu), enc.to(gpu), ga.to(gpu), stg.to(gpu), check=False)
    cache.check_rebuild()
    _check_cache(cache, want, want_lens)


@pytest.mark.parametrize("D", [128, 64])
def test_rebuild_any_layout_equals_cache_layout(gpu, D):
    """ma_rebuild_packed has an instantiation for stores laid out as the cache allocates
    them (constant strides inside a lane) and one reading every stride from the
    descriptor.  Old storage with padded inner dimensions (so the general one runs) and
    the cache's own layout give the oracle's bytes, bit for bit."""
    from maskahead_amd.kernels.rebuild import rebuild_packed
    from maskahead_amd.kernels.splitk import Prefix

    L, H, n_q, n_r = 2, 2, 1024, 32
    store, lens, g = _random_cache(31 + D, L=L, H=H, D=D, n_q=n_q, n_r=n_r)
    n = lens[0]
    gb = torch.tensor([[3, 7, 30], [0, 12, -1], [5, 6, 8], [31, 1, 2]]).view(L, 1, H, 3)
    enc = torch.stack([torch.randperm(n, generator=g)[:75].sort().values for _ in range(L * H)]).view(L, 1, H, 75)
    enc[1, 0, 1, 70:] = -1
    ga = torch.empty((L, 1, H, 0), dtype=torch.int64)
    stg = torch.stack([torch.randperm(n, generator=g)[:20].sort().values for _ in range(L * H)]).view(L, 1, H, 20)
    want, want_lens, want_remap = OR.rebuild(store, lens, gb, enc, ga, stg)
    nql, st = want_lens[1], want_lens[2]

    def planes(src, pad):
        """src (oracle layout) on the GPU; pad: dimension 4 widened (by 2 rows of codes or
        scales, by 8 residual channels, so rows stay as aligned as the library requires)
        and the original extent viewed: the same values, strides the cache never makes."""
        out = {}
        for short, _ in NAMES:
            t = src[short]
            if pad:
                w = 8 if short in ("kr", "vr") else 2
                big = torch.zeros([x + (w if i == 4 else 0) for i, x in enumerate(t.shape)], dtype=t.dtype)
                big[tuple(slice(0, x) for x in t.shape)] = t
                t = big.to(gpu)[tuple(slice(0, x) for x in t.shape)]
            else:
                t = t.to(gpu)
            out[short] = t
        return out

    def prefix(p, nq, nf):
        f = lambda x: p[x].flatten(0, 1)  # noqa: E731
        return Prefix(kq=f("kq"), ks=f("ks"), kz=f("kz"), vq=f("vq"), vs=f("vs"), vz=f("vz"), kf=f("kr"), vf=f("vr"),
                      nq=nq, nf=nf, kb=4, vb=4)

    empty = {"kq": torch.zeros((L, 1, H, nql // 32, D, 16), dtype=torch.uint8),
             "ks": torch.zeros((L, 1, H, nql // 32, D), dtype=torch.float16),
             "kz": torch.zeros((L, 1, H, nql // 32, D), dtype=torch.float16),
             "vq": torch.zeros((L, 1, H, nql, D // 32, 16), dtype=torch.uint8),
             "vs": torch.zeros((L, 1, H, nql, D // 32), dtype=torch.float16),
             "vz": torch.zeros((L, 1, H, nql, D // 32), dtype=torch.float16),
             "kr": torch.zeros((L, 1, H, st, D), dtype=torch.bfloat16),
             "vr": torch.zeros((L, 1, H, st, D), dtype=torch.bfloat16)}
    for pad in (True, False):
        old, new = planes(store, pad), planes(empty, False)
        remap = torch.empty((L, 1, H, n), dtype=torch.int64, device=gpu)
        assert (old["ks"].stride(4) == 1) and (old["ks"].stride(3) == (D + 2 if pad else D))
        rebuild_packed(prefix(old, n_q, n_r), prefix(new, nql, st), B=L, H=H, D=D, groups_before=gb.to(gpu),
                       encode=enc.to(gpu), groups_after=ga.to(gpu), stage=stg.to(gpu), remap=remap)
        torch.cuda.synchronize()
        for short, _ in NAMES:
            assert same_bits(new[short].cpu(), want[short]), (pad, short)
        assert torch.equal(remap.cpu(), want_remap), pad


def test_evict_to_bf16_cache_with_tail(gpu):
    """A 16-bit cache (session.py:292-296): the live slots, then a stored-but-unadmitted
    tail, gathered exactly in place; the state's slots become 0 .. live - 1."""
    from maskahead_amd.config import QuantizationConfig as QC

    L, H, D, n, tail, C = 2, 4, 64, 600, 40, 200
    g = torch.Generator().manual_seed(77)
    cache = PackedKVCache(num_layers=L, batch_size=1, num_kv_heads=H, head_dim=D, max_tokens=4096,
                          quant=QC(k_bits=16, v_bits=16), device=gpu)
    k = torch.randn((L, 1, H, n + tail, D), generator=g).to(torch.bfloat16)
    v = torch.randn((L, 1, H, n + tail, D), generator=g).to(torch.bfloat16)
    cache.begin_append(n + tail)
    for layer in range(L):
        cache.stage_layer(layer, k[layer].to(gpu), v[layer].to(gpu))
    cache.commit_append()
    st = EvictionState(num_layers=L, batch_size=1, num_kv_heads=H, capacity=n, device=gpu)
    st.append(range(n))
    keep = torch.stack([torch.randperm(n, generator=g)[:C].sort().values for _ in range(L * H)]).view(L, 1, H, C)
    cfg = EvictionConfig(policy="recent", recent_window=16, capacity_floor=16)
    evict_to(cache, st, keep.to(gpu), cfg, next_position=n)
    torch.cuda.synchronize()
    src = torch.cat([keep, torch.arange(n, n + tail).expand(L, 1, H, tail)], -1)
    gi = src.unsqueeze(-1).expand(-1, -1, -1, -1, D)
    assert cache.length == C + tail and cache.dropped == n - C
    assert same_bits(cache.k_fp[:, :, :, :C + tail], k.gather(3, gi))
    assert same_bits(cache.v_fp[:, :, :, :C + tail], v.gather(3, gi))
    assert torch.equal(st.phys[..., :C].cpu(), torch.arange(C, dtype=torch.int32).expand(L, 1, H, C))
