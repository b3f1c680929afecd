"""A session bound by runtime.bind.bind_session: the reference session's fast-path methods
(_fast_step0, _compact_attention, _fast_attend, _lookahead_evict, _evict_to, _live_values)
called as the reference's own code calls them, on a stand-in session that carries the
attributes and helper methods of BitSieveSession those methods read (session.py:97-200,
240-268, 438-454, 862-868).  Every result is bit-identical to the same stages called one by
one (splitk_attention, prefix_scores_topk, gather_packed_kv, lookahead_scores), the keep set
equals the oracle's, the eviction's side effects on the state and the trace are the
reference's, and attention after the eviction matches the oracle over the live entries."""

from __future__ import annotations

import contextlib
from dataclasses import dataclass
from types import SimpleNamespace

import pytest
import torch

from maskahead_amd.cache import PackedKVCache
from maskahead_amd.config import QuantizationConfig
from maskahead_amd.eviction import EvictionConfig, EvictionState
from maskahead_amd.kernels.ops import gather_packed_kv
from maskahead_amd.kernels.select import prefix_scores_topk
from maskahead_amd.kernels.splitk import Prefix, prefix_scores, splitk_attention
from maskahead_amd.runtime.bind import bind_session
from maskahead_amd.runtime.session import lookahead_scores
from maskahead_amd.workloads import layer_inputs
from oracle import attention as OA
from oracle import rebuild as OR
from oracle import selection as OS
from tests._util import assert_attention_close

pytestmark = pytest.mark.gpu


@dataclass
class SelectionRecord:
    block: int
    layer: int
    old_cache_len: int
    selected_k: int
    selector_queries: list
    semantic: str
    index_checksum: int


@dataclass
class CompactLayerState:
    key: torch.Tensor
    value: torch.Tensor
    indices: torch.Tensor | None = None
    selected_k: int = 0


class _Trace:
    def __init__(self):
        self.selections, self.counters = [], {}

    def add_counter(self, name, value):
        self.counters[name] = self.counters.get(name, 0) + value


class _Timer:
    def region(self, *args, **kwargs):
        return contextlib.nullcontext()


class _ForeignState:
    """An eviction state of another implementation, still empty (bind replaces it)."""

    def __init__(self, num_layers, batch_size, num_kv_heads, device):
        self.num_layers, self.batch_size, self.num_kv_heads, self.device = num_layers, batch_size, num_kv_heads, device
        self.live = 0


def _config(t, topk, cap, window, dense_layers):
    sel = SimpleNamespace(score="softmax", domain="prefix", mode="all", value_joint=False, value_per_query=False,
                          value_set="none", value_caote=False, value_aware=True, value_center="attn", topk=topk,
                          sort_indices=True, dense_prefix_layers=dense_layers)
    ev = EvictionConfig(policy="lookahead", recent_window=window, capacity_floor=cap, compaction="lazy",
                        repack_below=0.25)
    return SimpleNamespace(backend="auto", semantic="A", async_selector=False, collect_diagnostics=False,
                           coverage_diagnostics=False, compact_format="bf16", attn_log_dir=None, selector=sel,
                           eviction=ev, quant=QuantizationConfig(), generation=SimpleNamespace(block_size=t),
                           max_cache_tokens=1 << 20)


class _Session:
    """The members of BitSieveSession that its fast-path methods read, restated."""

    def __init__(self, cache, config, hkv, d):
        self.cache, self.config = cache, config
        self.num_kv_heads, self.head_dim, self.compute_dtype = hkv, d, torch.bfloat16
        self.trace, self.timer = _Trace(), _Timer()
        self.block_index = self.step_index = 0
        self.query_indices: list = []
        self.old_cache_len = 0
        self._states: dict = {}
        self._eviction = _ForeignState(cache.num_layers, cache.batch_size, hkv, cache.device)
        self._la_pending = None
        self._la_a1: dict = {}
        self._la_aprobe: dict = {}
        self._next_position = 0
        self._phys_compact = True
        self._attn_log = None

    @property
    def live_cache_len(self):
        return self._eviction.live

    def _live_positions(self, layer_idx):                      # session.py:236-238
        st = self._eviction
        return st.phys[layer_idx, ..., :st.live].to(torch.int64)

    def _slot_mask(self, layer_idx):                           # session.py:240-255
        st = self._eviction
        if self.cache.length <= st.live:
            return None
        key = (getattr(self, "_mask_epoch", 0), self.cache.length, st.live)
        cached = getattr(self, "_mask_cache", None)
        if cached is None or cached[0] != key:
            cached = self._mask_cache = (key, {})
        m = cached[1].get(layer_idx)
        if m is None:
            m = torch.zeros((self.cache.batch_size, self.num_kv_heads, self.cache.length), dtype=torch.uint8,
                            device=self.cache.device)
            m.scatter_(-1, self._live_positions(layer_idx), 1)
            cached[1][layer_idx] = m
        return m

    def _to_live(self, layer_idx, per_slot):                   # session.py:257-261
        return per_slot.gather(-1, self._live_positions(layer_idx))

    def _effective_budget(self):                               # session.py:862-868
        return min(self.config.selector.topk, self.live_cache_len)

    def _ensure_state(self, layer_idx, selected_k):            # session.py:438-454
        state = self._states.get(layer_idx)
        capacity = max(1, selected_k) + self.config.generation.block_size
        if state is not None and state.key.shape[2] >= capacity:
            return state
        shape = (self.cache.batch_size, self.num_kv_heads, capacity, self.head_dim)
        state = CompactLayerState(key=torch.empty(shape, device=self.cache.device, dtype=torch.bfloat16),
                                  value=torch.empty(shape, device=self.cache.device, dtype=torch.bfloat16))
        self._states[layer_idx] = state
        return state

    def _lookahead_evict(self, capacity):
        raise AssertionError("the bound session must not take the torch lookahead path")

    def _log_score(self, score, source, capacity):
        pass

    def _log_pairwise_eviction(self, capacity):
        pass


def _snapshot(cache):
    names = (("kq", "k_q"), ("ks", "k_scale"), ("kz", "k_zero"), ("vq", "v_q"), ("vs", "v_scale"), ("vz", "v_zero"),
             ("kr", "k_residual"), ("vr", "v_residual"))
    lens = (cache.length, cache.quantized_length, cache.residual_length, cache.dropped)
    return {short: getattr(cache, name).cpu() for short, name in names}, lens


def test_bound_session_block_cycle(gpu):
    L, hq, hkv, d, n, t, k, C, W = 3, 28, 4, 128, 4096, 32, 512, 1024, 64
    q, kk, v, kc, vc = layer_inputs(b=1, hq=hq, hkv=hkv, d=d, n=n, t=t, seed=61, dtype=torch.bfloat16)
    cache = PackedKVCache(num_layers=L, batch_size=1, num_kv_heads=hkv, head_dim=d, max_tokens=1 << 16,
                          quant=QuantizationConfig(), device=gpu)
    s = _Session(cache, _config(t, k, C, W, dense_layers=1), hkv, d)
    fp = bind_session(s)
    assert isinstance(s._eviction, EvictionState) and fp.states is s._states
    cache.begin_append(n)
    for layer in range(L):
        cache.stage_layer(layer, (kk + layer).to(gpu), v.to(gpu))
    cache.commit_append()
    st = s._eviction
    st.append(range(n))
    s._next_position = n
    s.query_indices, s._la_pending, s.old_cache_len = list(range(t)), C, n
    qg, kcg, vcg = q.to(gpu), kc.to(gpu), vc.to(gpu)

    # step 0 of every layer: layer 0 dense (attention + mass), the others sparse (read set)
    for layer in range(L):
        dense = layer < 1
        out = s._fast_step0(layer, qg, kcg, vcg, dense)
        pre = Prefix.from_view(cache.layer_view(layer))
        wout, stats = splitk_attention(qg, pre, kcg, vcg, want_prefix=True)
        torch.cuda.synchronize()
        assert torch.equal(out, wout)
        if dense:
            wmass, _ = prefix_scores(qg, pre, stats, list(range(t)), value=False)
            assert layer not in s._states
        else:
            wmass, _, widx = prefix_scores_topk(qg, pre, stats, list(range(t)), k, value=True)
            ck, cv = gather_packed_kv(pre, widx)
            state = s._states[layer]
            assert state.selected_k == k and torch.equal(state.indices, widx)
            assert torch.equal(state.key[:, :, :k], ck) and torch.equal(state.value[:, :, :k], cv)
        assert torch.equal(s._la_a1[layer], wmass)                # live order = slot order here
    assert [r.layer for r in s.trace.selections] == [1, 2]
    assert all(r.selected_k == k and r.old_cache_len == n for r in s.trace.selections)

    # a denoising sub-step of a sparse layer: [read set | block]
    g = torch.Generator().manual_seed(62)
    q2, kc2, vc2 = (torch.randn(shape, generator=g).to(torch.bfloat16)
                    for shape in ((1, hq, t, d), (1, hkv, t, d), (1, hkv, t, d)))
    state = s._states[2]
    out2 = s._compact_attention(2, q2.to(gpu), kc2.to(gpu), vc2.to(gpu))
    want2, _ = splitk_attention(q2.to(gpu), Prefix.dense(state.key[:, :, :k], state.value[:, :, :k]), kc2.to(gpu),
                                vc2.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(out2, want2)
    assert_attention_close(out2, OA.dense_attention(q2, state.key[:, :, :k].cpu(), state.value[:, :, :k].cpu(),
                                                    kc2, vc2))

    # the lookahead eviction at the end of step 0: keep set = the oracle's on the same score
    score = lookahead_scores(cache, st, s._la_a1, s._la_aprobe, use_value=True)
    pos0 = st.pos[..., :n].cpu().to(torch.int64)
    want_keep = OS.keep_select(pos0, score.cpu(), C, W)
    s._lookahead_evict(C)
    torch.cuda.synchronize()
    assert st.live == C and torch.equal(st.pos[..., :C].cpu().to(torch.int64), pos0.gather(-1, want_keep))
    assert s.trace.counters == {"evictions": 1, "entries_evicted": n - C}
    assert s._mask_epoch == 1 and cache.length > C            # kept groups carry dead slots

    # the next block over the rebuilt cache: the bound prefix carries the live mask, the
    # live values come from the codes
    store, lens = _snapshot(cache)
    kd, vd = OR._dequantize_all(store, lens)
    q3, kc3, vc3 = (torch.randn(shape, generator=g).to(torch.bfloat16)
                    for shape in ((1, hq, t, d), (1, hkv, t, d), (1, hkv, t, d)))
    for layer in range(L):
        phys = st.phys[layer, ..., :C].cpu().to(torch.int64)
        out3, mass3 = s._fast_attend(layer, q3.to(gpu), kc3.to(gpu), vc3.to(gpu), mass_rows=list(range(t)))
        gi = phys.unsqueeze(-1).expand(-1, -1, -1, d)
        kl, vl = kd[layer].gather(2, gi), vd[layer].gather(2, gi)
        assert_attention_close(out3, OA.dense_attention(q3, kl, vl, kc3, vc3))
        assert torch.equal(s._live_values(layer).cpu(), vl)
        dead = s._slot_mask(layer).cpu() == 0
        assert dead.any() and (mass3.cpu()[dead] == 0).all()
