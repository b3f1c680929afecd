"""The drop-in boundary by member: every attribute the reference's runtime modules read or
call on a KV-cache object or an eviction-state object (listed from the reference's own
source by tests/golden/make_import_names.py, with file:line) exists on
maskahead_amd.cache.PackedKVCache and maskahead_amd.eviction.EvictionState, and the
accounting members that need no GPU (state_nbytes, live_cache_nbytes, the sink-eviction
counters) agree with brute-force counts.  No kernel runs here: caches and states are
built on the CPU."""

import json
from pathlib import Path

import pytest
import torch

import maskahead_amd.cache as C
import maskahead_amd.eviction as E
from maskahead_amd.config import QuantizationConfig

FIX = json.loads((Path(__file__).resolve().parent / "golden" / "reference_kernel_imports.json").read_text())


@pytest.mark.parametrize("quant", [QuantizationConfig(), QuantizationConfig(k_bits=16, v_bits=16)],
                         ids=["k4v4", "bf16"])
def test_cache_has_every_member_the_runtime_uses(quant):
    cache = C.PackedKVCache(num_layers=2, batch_size=1, num_kv_heads=2, head_dim=128, max_tokens=256, quant=quant,
                            device="cpu")
    used = FIX["attributes"]["cache"]
    assert {"load_dynamic_cache", "layer_view", "begin_append", "logical_nbytes"} <= set(used)
    missing = {a: w for a, w in used.items() if not hasattr(cache, a)}
    assert not missing, f"cache members the reference runtime uses but maskahead_amd lacks: {missing}"


def test_eviction_state_has_every_member_the_runtime_uses():
    st = E.EvictionState(num_layers=2, batch_size=1, num_kv_heads=2, capacity=8, device="cpu")
    used = FIX["attributes"]["eviction_state"]
    assert {"state_nbytes", "maybe_evict", "observe", "live"} <= set(used)
    missing = {a: w for a, w in used.items() if not hasattr(st, a)}
    assert not missing, f"eviction-state members the reference runtime uses but maskahead_amd lacks: {missing}"
    for a in FIX["assigned"]["eviction_state"]:      # assigned by the runtime: settable
        setattr(st, a, getattr(st, a, None))


def _state(lanes_pos: torch.Tensor) -> E.EvictionState:
    l, b, h, n = lanes_pos.shape
    st = E.EvictionState(num_layers=l, batch_size=b, num_kv_heads=h, capacity=n, device="cpu")
    st.append(range(n))
    st.pos[..., :n] = lanes_pos.to(st.pos.dtype)
    return st


def test_state_nbytes_counts_ema_count_and_position_per_live_entry():
    st = E.EvictionState(num_layers=3, batch_size=2, num_kv_heads=4, capacity=10, device="cpu",
                         max_position=1 << 20)
    assert st.state_nbytes() == 0
    st.append(range(7))
    assert st.state_nbytes() == 3 * 2 * 4 * 7 * (4 + 2 + 4)   # f32 EMA, int16 count, int32 position
    wide = E.EvictionState(num_layers=1, batch_size=1, num_kv_heads=1, capacity=4, device="cpu")
    wide.append(range(3))                                    # the default max_position 2^31 needs int64
    assert wide.state_nbytes() == 3 * (4 + 2 + 8)


@pytest.mark.parametrize("kb,vb", [(4, 4), (16, 16), (4, 16), (16, 4)])
def test_live_cache_nbytes_against_brute_force(kb, vb):
    g = torch.Generator().manual_seed(7)
    l, b, h, rows, live, d = 2, 2, 3, 300, 220, 128
    pos = torch.zeros(l, b, h, rows, dtype=torch.int32)
    for lane in range(l * b * h):           # each lane: a scattered, unsorted live set of distinct positions
        pos.view(-1, rows)[lane, :live] = torch.randperm(2000, generator=g)[:live].to(torch.int32)
    got = E.live_cache_nbytes(pos, live=live, head_dim=d, k_bits=kb, v_bits=vb, key_token_group=32,
                              value_channel_group=32, param_bytes=2, compute_bytes=2)
    groups = sum(len({int(p) // 32 for p in row[:live]}) for row in pos.view(-1, rows))
    entries = l * b * h * live
    want_k = entries * d * 2 if kb == 16 else entries * d // 2 + groups * d * 2 * 2
    want_v = entries * d * 2 if vb == 16 else entries * d // 2 + entries * (d // 32) * 2 * 2
    assert got == want_k + want_v
    assert E.live_cache_nbytes(pos, live=0, head_dim=d, k_bits=kb, v_bits=vb, key_token_group=32,
                               value_channel_group=32) == 0
    # a contiguous run of 64 positions occupies two key groups per lane
    run = torch.arange(64, dtype=torch.int32).view(1, 1, 1, 64).expand(1, 1, 2, 64).contiguous()
    assert E.live_cache_nbytes(run, live=64, head_dim=d, k_bits=4, v_bits=4, key_token_group=32,
                               value_channel_group=32) == 2 * (64 * 64 + 2 * d * 4 + 64 * 64 + 64 * 4 * 4)


def test_sink_eviction_counters():
    # lanes: positions 0..9; keep sets that keep all, some or none of the sinks 0..3
    pos = torch.arange(10, dtype=torch.int32).view(1, 1, 1, 10).expand(2, 1, 3, 10).contiguous()
    st = _state(pos)
    assert st.sink_lanes_evicted == 0 and st.lanes_evictions == 0
    keep = torch.tensor([[[[0, 1, 2, 3, 9]], [[0, 1, 2, 8, 9]], [[5, 6, 7, 8, 9]]],
                         [[[0, 1, 2, 3, 4]], [[1, 2, 3, 4, 5]], [[0, 1, 2, 3, 6]]]]).view(2, 1, 3, 5)
    st._count_sink_drops(keep)
    want = sum(int(any(p < 4 and p not in set(row.tolist()) for p in range(10))) for row in keep.view(-1, 5))
    assert want == 3 and st.sink_lanes_evicted == 3 and st.lanes_evictions == 6
    st._count_sink_drops(keep)
    assert st.sink_lanes_evicted == 6 and st.lanes_evictions == 12
