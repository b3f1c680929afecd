"""Host-side logic of the cache and fast-path mirrors (no GPU): quantization settings and
their validation (config.py:28-86), the append plan and storage layouts of
PackedKVCache (cache.py:63-189, 385-421), the read budget (config.py:172-183) and the
fast-path routing conditions (session.py:43-75)."""

from types import SimpleNamespace

import pytest
import torch

from maskahead_amd._native import KernelUnavailableError
from maskahead_amd.cache import PackedKVCache
from maskahead_amd.config import QuantizationConfig
from maskahead_amd.runtime.fastpath import effective_topk, fast_path_supported


def test_quantization_validate_messages():
    with pytest.raises(ValueError, match="k_bits must be 2, 4, or 16; got 3"):
        QuantizationConfig(k_bits=3).validate()
    with pytest.raises(ValueError, match="key_token_group must be a positive multiple of 8"):
        QuantizationConfig(key_token_group=12).validate()
    with pytest.raises(ValueError, match="head_dim=100 must be divisible"):
        QuantizationConfig().validate(head_dim=100)
    QuantizationConfig().validate(head_dim=128)
    with pytest.raises(KernelUnavailableError):
        QuantizationConfig(k_bits=2, v_bits=2).require_built()
    with pytest.raises(KernelUnavailableError):
        QuantizationConfig(key_mode="token").require_built()
    QuantizationConfig(k_bits=16, v_bits=16, key_token_group=8).require_built()


def test_cache_layouts_and_append_plan_cpu():
    c = PackedKVCache(num_layers=3, batch_size=2, num_kv_heads=4, head_dim=128, max_tokens=5000,
                      quant=QuantizationConfig(), device="cpu")
    cap, rcap = c.capacity, c.residual_capacity
    assert cap % 32 == 0 and 32 <= cap <= 5024 and rcap >= 32 + 32    # a whole block beyond the residual fits
    assert tuple(c.k_q.shape) == (3, 2, 4, cap // 32, 128, 16) and tuple(c.k_scale.shape) == (3, 2, 4, cap // 32, 128)
    assert tuple(c.v_q.shape) == (3, 2, 4, cap, 4, 16) and tuple(c.v_scale.shape) == (3, 2, 4, cap, 4)
    assert c.k_scale.dtype == torch.float16 and c.k_fp is None
    assert tuple(c.k_residual.shape) == (3, 2, 4, rcap, 128) and c.k_residual.dtype == torch.bfloat16
    plan = c.begin_append(1000)
    assert (plan.quantize_from_residual, plan.new_residual) == (960, 40)
    with pytest.raises(RuntimeError, match="already in progress"):
        c.begin_append(1)
    c.abort_append()
    plan = c.begin_append(4000)                       # grows the storage past its first allocation
    assert c.capacity >= 4000 and c.k_q.shape[3] == c.capacity // 32 and c.v_q.shape[3] == c.capacity
    assert (plan.quantize_from_residual, plan.new_residual) == (3968, 32)
    with pytest.raises(ValueError, match="shape mismatch"):
        c.stage_layer(0, torch.zeros(2, 4, 3, 128), torch.zeros(2, 4, 3, 128))
    with pytest.raises(RuntimeError, match="not staged"):
        c.commit_append()
    c.abort_append()
    with pytest.raises(RuntimeError, match="capacity exceeded"):
        c.begin_append(6000)
    b = PackedKVCache(num_layers=1, batch_size=1, num_kv_heads=2, head_dim=64, max_tokens=100,
                      quant=QuantizationConfig(k_bits=16, v_bits=16), device="cpu")
    assert b.capacity >= 100 and tuple(b.k_fp.shape) == (1, 1, 2, b.capacity, 64) and b.k_q is None
    assert b.residual_capacity == 0 and b.k_residual is None
    # accounting: nothing in use yet; every plane's bytes allocated
    assert c.logical_nbytes()["total"] == 0
    # in use: the rows of each plane's unit (whole key groups, quantized tokens, residual),
    # counted as the bytes of those rows' slices
    c.length, c.quantized_length, c.residual_length = 1000, 960, 40
    want = {}
    for name, part in (("k_q", "key_payload"), ("k_scale", "key_metadata"), ("k_zero", "key_metadata"),
                       ("k_residual", "key_residual"), ("v_q", "value_payload"), ("v_scale", "value_metadata"),
                       ("v_zero", "value_metadata"), ("v_residual", "value_residual")):
        t = getattr(c, name)
        rows = {"k_q": 30, "k_scale": 30, "k_zero": 30, "k_residual": 40}.get(name, 960 if "residual" not in name else 40)
        want[part] = want.get(part, 0) + t[:, :, :, :rows].numel() * t.element_size()
    got = c.logical_nbytes()
    assert all(got[x] == want[x] for x in want) and got["total"] == sum(want.values())
    c.length = c.quantized_length = c.residual_length = 0
    assert c.allocated_nbytes() == sum(t.numel() * t.element_size() for t in (c.k_q, c.k_scale, c.k_zero, c.v_q,
                                                                               c.v_scale, c.v_zero, c.k_residual,
                                                                               c.v_residual))
    with pytest.raises(KernelUnavailableError):
        PackedKVCache(num_layers=1, batch_size=1, num_kv_heads=2, head_dim=64, max_tokens=100,
                      quant=QuantizationConfig(), device="cpu", backend="torch")


def test_effective_topk():
    assert effective_topk(0, 512) == 0
    assert effective_topk(300, 512) == 300
    assert effective_topk(4096, 512) == 512
    assert effective_topk(4096, 512, topk_percent=10.0) == 410
    assert effective_topk(50, 512, topk_percent=1.0, topk_floor=16) == 16


def _cfg(**over):
    sel = SimpleNamespace(score="softmax", domain="prefix", mode="all", value_joint=False, value_per_query=False,
                          value_set="none", value_caote=False, value_aware=True, value_center="attn")
    ev = SimpleNamespace(enabled=False, policy="lookahead", diag_path=None, oracle_record_dir=None)
    q = QuantizationConfig()
    cfg = SimpleNamespace(backend="auto", semantic="A", async_selector=False, collect_diagnostics=False,
                          coverage_diagnostics=False, compact_format="bf16", attn_log_dir=None,
                          selector=sel, eviction=ev, quant=q)
    for k, v in over.items():
        obj, _, attr = k.rpartition("__")
        setattr(getattr(cfg, obj) if obj else cfg, attr, v)
    return cfg


def test_fast_path_supported_reasons():
    assert fast_path_supported(_cfg(), 128) == (True, "head_dim")
    assert fast_path_supported(_cfg(), 96) == (False, "head_dim")
    assert fast_path_supported(_cfg(), 128, "cpu")[1] == "disabled or not cuda"
    assert fast_path_supported(_cfg(backend="torch"), 128)[1] == "backend/semantic"
    assert fast_path_supported(_cfg(compact_format="requantized"), 128)[1] == "diagnostics/compact format"
    assert fast_path_supported(_cfg(selector__mode="uniform"), 128)[1] == "selector score/domain/mode"
    assert fast_path_supported(_cfg(selector__value_center="mean"), 128)[1] == "value centre"
    assert fast_path_supported(_cfg(quant=QuantizationConfig(k_bits=2, v_bits=2)), 128)[1] == "bits"
    assert fast_path_supported(_cfg(quant=QuantizationConfig(key_token_group=16)), 128)[1] == "group sizes"
    assert fast_path_supported(_cfg(quant=QuantizationConfig(k_bits=16, v_bits=16)), 64) == (True, "head_dim")


def _bind_target(cfg, head_dim=128):
    """A session-shaped object with the members bind_session reads at bind time."""
    class Session:
        def _fast_step0(self, *a):
            return "reference"

        def _compact_attention(self, *a):
            return "reference"

    s = Session()
    cfg.selector.sort_indices, cfg.selector.dense_prefix_layers = True, 0
    cfg.generation = SimpleNamespace(block_size=32)
    s.config, s.head_dim, s.compute_dtype, s._states, s._eviction = cfg, head_dim, torch.bfloat16, {}, None
    s.cache = SimpleNamespace(device=torch.device("cuda"))
    return s


def test_bind_session_host():
    """bind_session refuses a configuration the HIP path does not serve and leaves the
    session as it was; otherwise it replaces the fast-path methods on that instance only,
    the class and the session's compact states left shared."""
    from maskahead_amd.runtime.bind import bind_session, bind_value_score

    s = _bind_target(_cfg(selector__mode="uniform"))
    with pytest.raises(KernelUnavailableError, match="selector score/domain/mode"):
        bind_session(s)
    assert s._fast_step0() == "reference" and "_fast_step0" not in vars(s)
    s = _bind_target(_cfg(), head_dim=96)
    with pytest.raises(KernelUnavailableError, match="head_dim"):
        bind_session(s)

    s = _bind_target(_cfg())
    fp = bind_session(s)
    for name in ("_fast_step0", "_compact_attention", "_fast_attend", "_current_only", "_prefix", "_live_values"):
        assert name in vars(s), name
    assert "_evict_to" not in vars(s)                 # another cache type keeps its own eviction
    assert fp.states is s._states and fp.block_size == 32 and fp.value_aware
    assert type(s)()._fast_step0() == "reference"

    mod = SimpleNamespace(value_score=lambda a, v: None)
    old = bind_value_score(mod)
    from maskahead_amd.runtime.session import value_score

    assert mod.value_score is value_score and old is not value_score


def test_batch_fast_path_checks_its_caches():
    """BatchFastPath takes one single-sequence cache per sequence, all of one head shape."""
    from maskahead_amd.runtime.batch import BatchFastPath

    def cache(d=128, b=1):
        return PackedKVCache(num_layers=2, batch_size=b, num_kv_heads=4, head_dim=d, max_tokens=256,
                             quant=QuantizationConfig(), device="cpu")

    with pytest.raises(ValueError):
        BatchFastPath([], block_size=32)
    with pytest.raises(ValueError):
        BatchFastPath([cache(), cache(d=64)], block_size=32)
    with pytest.raises(ValueError):
        BatchFastPath([cache(b=2)], block_size=32)
    bp = BatchFastPath([cache(), cache()], block_size=32, query_indices=range(32), dense_prefix_layers=1)
    assert bp.batch_size == 2 and all(p.dense_prefix_layers == 1 for p in bp.paths)


def test_admitting_entries_after_a_compaction():
    """After a compaction the slots of newly committed entries are the cache's newest
    physical slots, not their positions (session.py:215-229); live_slot_masks refuses a
    state whose slots lie outside the cache instead of scattering out of bounds."""
    from maskahead_amd.eviction import EvictionState
    from maskahead_amd.runtime.session import admit_new_entries, live_slot_masks

    cache = PackedKVCache(num_layers=2, batch_size=1, num_kv_heads=2, head_dim=128, max_tokens=4096,
                          quant=QuantizationConfig(), device="cpu")
    st = EvictionState(num_layers=2, batch_size=1, num_kv_heads=2, capacity=64, device="cpu")
    # a cache that held 1000 positions, compacted to 300 physical slots, then 32 appended
    cache.length, cache.dropped = 332, 700
    st.append(range(250), phys=torch.arange(250) + 40)          # survivors in slots 40 .. 289
    assert admit_new_entries(cache, st, 1000) == 1032
    assert st.live == 282
    assert torch.equal(st.pos[0, 0, 0, 250:282].long(), torch.arange(1000, 1032))
    assert torch.equal(st.phys[0, 0, 0, 250:282].long(), torch.arange(300, 332))
    masks = live_slot_masks(cache, st)
    assert int(masks[0].sum()) == 2 * 282 and int(masks[1][0, 1, :40].sum()) == 0
    assert admit_new_entries(cache, st, 1032) == 1032 and st.live == 282     # nothing new
    wrong = EvictionState(num_layers=2, batch_size=1, num_kv_heads=2, capacity=64, device="cpu")
    wrong.append(range(1000, 1032))                               # positions as slots
    with pytest.raises(ValueError, match="outside the cache"):
        live_slot_masks(cache, wrong)


def test_rows_contiguous():
    """The per-plane row check of compact_tokens: the dims after the token axis must form
    one contiguous row; dims of size 1 place no constraint."""
    from maskahead_amd.kernels.keep import _rows_contiguous

    t = torch.zeros(2, 3, 10, 4, 5)
    assert _rows_contiguous(t.shape[3:], t.stride()[3:])
    assert _rows_contiguous((), ())
    tt = t.transpose(3, 4)
    assert not _rows_contiguous(tt.shape[3:], tt.stride()[3:])
    assert _rows_contiguous((1, 5), (999, 1))
    s = t[..., ::2]
    assert not _rows_contiguous(s.shape[3:], s.stride()[3:])


def test_rebuild_plan_cut_host():
    """The plan's lists are cut to the largest count of any lane (groups, encoded, staged)
    from the counts read back to the host; a negative count (a lane the plan could not
    order) raises KernelUnavailableError."""
    from maskahead_amd.kernels.rebuild import rebuild_plan_cut

    lead = (2, 1, 2)
    gb = torch.arange(4 * 10).view(4, 10)
    enc = torch.arange(4 * 50).view(4, 50)
    stg = torch.arange(4 * 50).view(4, 50) + 1000
    counts = torch.tensor([[3, 40, 0], [7, 12, 5], [1, 0, 2], [0, 33, 1]], dtype=torch.int32)
    g, e, s = rebuild_plan_cut((gb, enc, stg, None, lead), counts)
    assert g.shape == (2, 1, 2, 7) and e.shape == (2, 1, 2, 40) and s.shape == (2, 1, 2, 5)
    assert torch.equal(g.reshape(4, 7), gb[:, :7]) and torch.equal(s.reshape(4, 5), stg[:, :5])
    counts[2, 1] = -1
    with pytest.raises(KernelUnavailableError):
        rebuild_plan_cut((gb, enc, stg, None, lead), counts)
    empty = rebuild_plan_cut((gb[:0], enc[:0], stg[:0], None, (0, 1, 2)), counts[:0])
    assert all(t.shape == (0, 1, 2, 0) for t in empty)
