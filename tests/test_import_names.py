"""The drop-in boundary by name: every name the reference package imports from the
modules this package replaces (maskahead.kernels.ops, maskahead.kernels.splitk,
maskahead.cache, maskahead.eviction; list written from
the reference's own import statements by tests/golden/make_import_names.py) exists in
the matching maskahead_amd module, so re-exporting these modules under the reference's
paths leaves no import of the session, cache or generators unresolved."""

import importlib
import json
from pathlib import Path

import pytest

NAMES = json.loads((Path(__file__).resolve().parent / "golden" / "reference_kernel_imports.json").read_text())


MODULES = {"ops": "maskahead_amd.kernels.ops", "splitk": "maskahead_amd.kernels.splitk",
           "cache": "maskahead_amd.cache", "eviction": "maskahead_amd.eviction"}


@pytest.mark.parametrize("short", sorted(MODULES))
def test_every_imported_kernel_name_exists(short):
    mod = importlib.import_module(MODULES[short])
    names = NAMES["names"][short]
    assert names, "the fixture lists no names"
    missing = {n: where for n, where in names.items() if not hasattr(mod, n)}
    assert not missing, f"names the reference imports from {short} but maskahead_amd lacks: {missing}"


def test_fixture_covers_the_fast_path_imports():
    # the session's fast probe branch imports _selected_queries (session.py:2321, 2343)
    where = NAMES["names"]["ops"]["_selected_queries"]
    assert any(w.startswith("src/maskahead/runtime/session.py:") for w in where)
    assert set(NAMES["names"]["splitk"]) >= {"Prefix", "splitk_attention", "prefix_scores"}
