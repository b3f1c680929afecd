"""The C ABI: the built library loads and exports every symbol include/maskahead_hip.h
declares, the ctypes table matches the header, and argument errors map to the
reference's exception types -- all without launching a kernel (no GPU needed)."""

import re
from pathlib import Path

import pytest

from maskahead_amd import _native as N

HEADER = Path(__file__).resolve().parents[1] / "include" / "maskahead_hip.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ma_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not N.LIB_PATH.exists():
        from maskahead_amd.build import build

        build()
    return N.load()


def test_header_declares_the_path():
    names = _declared()
    for required in ("ma_dequant_prefix", "ma_splitk_attention", "ma_prefix_scores", "ma_topk_select",
                     "ma_gather_kv", "ma_quantize_keys", "ma_quantize_values"):
        assert required in names


def test_every_declared_symbol_is_exported(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_ctypes_table_matches_header():
    assert sorted(N.SIGNATURES) == _declared()


def test_version_and_error_mapping(lib):
    assert lib.ma_version() >= 1
    # k > n: rejected on the host before any launch
    rc = lib.ma_topk_select(1, 8, None, 0, 1, 8, 9, 1, 9, None, None, 0, None, 0, None)
    assert rc == N.MA_EINVAL
    assert b"bad arguments" in lib.ma_last_error()
    with pytest.raises(ValueError):
        N.check(rc, "ma_topk_select")
    with pytest.raises(N.KernelUnavailableError):
        N.check(N.MA_EUNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        N.check(N.MA_EHIP, "x")


def test_unsupported_prefix_is_reported(lib):
    p = N.MaPrefix()
    p.nq, p.kbits, p.vbits, p.kgroup, p.vgroup = 32, 2, 2, 32, 32
    rc = lib.ma_gather_kv(p, 1, 1, 128, 1, N.i64arr(0, 0), 1, N.MaTensor4(), N.MaTensor4(), None)
    assert rc == N.MA_EUNSUPPORTED
    assert b"bit widths" in lib.ma_last_error()
    rc = lib.ma_splitk_attention(N.MaTensor4(), 1, 28, 32, 96, p, 4, N.MaTensor4(), N.MaTensor4(), 0, 0, 0, 0,
                                 1.0, N.MaTensor4(), None, None, None, 0, None, 0, None)
    assert rc == N.MA_EUNSUPPORTED          # head_dim 96 is not built


def test_rebuild_arguments_are_checked_on_the_host(lib):
    """ma_rebuild_plan / ma_rebuild_packed reject bad sizes before any launch."""
    # window larger than the live count
    rc = lib.ma_rebuild_plan(1, 8, 1, 0, 8, 1, 4, 64, 16, 0, 5, 1, 2, 1, 8, 1, 8, 1, None)
    assert rc == N.MA_EINVAL and b"bad sizes" in lib.ma_last_error()
    # quantized length not a multiple of the key group
    rc = lib.ma_rebuild_plan(1, 8, 1, 0, 8, 1, 4, 40, 16, 0, 0, 1, 2, 1, 8, 1, 8, 1, None)
    assert rc == N.MA_EINVAL
    # more key groups than the plan counts in LDS
    rc = lib.ma_rebuild_plan(1, 8, 1, 0, 8, 1, 4, 32 * 40000, 16, 0, 0, 1, 40000, 1, 8, 1, 8, 1, None)
    assert rc == N.MA_EUNSUPPORTED
    # no old storage; then new storage whose length disagrees with the lists
    rc = lib.ma_rebuild_packed(None, 1, 1, 64, None, None, 0, 0, None, 0, 0, None, 0, 0, None, 0, 0, None, 0,
                               None, 0, 0, None, None)
    assert rc == N.MA_EINVAL
    old, new = N.MaPrefix(), N.MaPrefix()
    rc = lib.ma_rebuild_packed(old, 1, 1, 64, new, None, 0, 1, None, 0, 0, None, 0, 0, None, 0, 0, None, 0,
                               None, 0, 0, None, None)   # one kept group, but new storage of 0 entries
    assert rc == N.MA_EINVAL and b"expected" in lib.ma_last_error()


def test_fused_score_select_arguments_are_checked_on_the_host(lib):
    """The score pass with the select's first histogram level and the select that uses it
    reject bad arguments before any launch; the Python pair rejects a bad rank."""
    rc = lib.ma_prefix_scores_hist(N.MaTensor4(), 1, 28, 32, 128, N.MaPrefix(), 4, None, 32, None, None, None, 0,
                                   1.0, 1, 0, None, None, 3, None, 0, None)
    assert rc == N.MA_EINVAL and b"rank must be" in lib.ma_last_error()
    rc = lib.ma_topk_select_hist_ready(None, 0, None, 0, -1, 10, 1, None, 1, None, None, 0, None, 0, None)
    assert rc == N.MA_EINVAL and b"bad arguments" in lib.ma_last_error()
    from maskahead_amd.kernels import prefix_scores_topk

    with pytest.raises(ValueError):
        prefix_scores_topk(None, None, (None, None, None, None), [0], 1, value=False, rank="score")
    with pytest.raises(ValueError):
        prefix_scores_topk(None, None, (None, None, None, None), [0], 1, value=True, rank="keys")


def test_packed_append_arguments_are_checked_on_the_host(lib):
    """ma_append_packed rejects a split that is not whole key groups, a count that does not
    add up, and mixed dtypes, before any launch."""
    def t4(dtype=N.MA_BF16, ptr=16):
        m = N.MaTensor4()
        m.ptr, m.dtype = ptr, dtype
        return m

    z3, z4 = N.i64arr(0, 0, 0), N.i64arr(0, 0, 0, 0)
    # move not a multiple of 32
    rc = lib.ma_append_packed(t4(), t4(), 8, t4(), t4(), 1, 4, 32, 128, 16, 24, None, z4, None, None, z3, None, z4,
                              None, None, z3, None)
    assert rc == N.MA_EINVAL and b"move % 32" in lib.ma_last_error()
    # move + keep != old_res + T
    rc = lib.ma_append_packed(t4(), t4(), 8, t4(), t4(), 1, 4, 32, 128, 32, 16, None, z4, None, None, z3, None, z4,
                              None, None, z3, None)
    assert rc == N.MA_EINVAL
    # residual in f32, new tokens in bf16
    rc = lib.ma_append_packed(t4(N.MA_F32), t4(N.MA_F32), 8, t4(), t4(), 1, 4, 32, 128, 0, 40, None, z4, None, None,
                              z3, None, z4, None, None, z3, None)
    assert rc == N.MA_EINVAL and b"dtype" in lib.ma_last_error()
    # quantizing with no planes
    rc = lib.ma_append_packed(t4(), t4(), 0, t4(), t4(), 1, 4, 32, 128, 32, 0, None, z4, None, None, z3, None, z4,
                              None, None, z3, None)
    assert rc == N.MA_EINVAL and b"planes" in lib.ma_last_error()
