"""The CPU oracle against the golden vectors written by the reference itself
(tests/golden/make_golden.py): the bf16 keep score and the 4-bit quantizers."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as OA

GOLD = Path(__file__).resolve().parent / "golden" / "golden_vectors.npz"


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def _bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("tag", ["vs_small", "vs_mid"])
def test_value_score_bf16_matches_reference(gold, tag):
    a = torch.from_numpy(gold[f"{tag}_a"])
    v = _bf16(gold[f"{tag}_v"])
    want = torch.from_numpy(gold[f"{tag}_score"])
    got = OA.value_score_bf16(a, v)
    # every rounding point of session.py:38-40 is reproduced: bit-exact
    assert torch.equal(got, want), ((got - want).abs() / want.abs().clamp_min(1e-30)).max()


@pytest.mark.parametrize("tag", ["bf16", "f32"])
def test_quantizers_match_reference(gold, tag):
    x = gold[f"q_{tag}_x"]
    xt = _bf16(x) if tag == "bf16" else torch.from_numpy(x)
    kq, ks, kz = OA.quantize_keys(xt)
    vq, vs, vz = OA.quantize_values(xt)
    assert np.array_equal(kq.numpy(), gold[f"q_{tag}_kq"])
    assert np.array_equal(ks.view(torch.int16).numpy().view(np.uint16), gold[f"q_{tag}_ks"])
    assert np.array_equal(kz.view(torch.int16).numpy().view(np.uint16), gold[f"q_{tag}_kz"])
    assert np.array_equal(vq.numpy(), gold[f"q_{tag}_vq"])
    assert np.array_equal(vs.view(torch.int16).numpy().view(np.uint16), gold[f"q_{tag}_vs"])
    assert np.array_equal(vz.view(torch.int16).numpy().view(np.uint16), gold[f"q_{tag}_vz"])


@pytest.mark.parametrize("tag", ["lazy", "lazy2", "full", "stage", "tail"])
def test_rebuild_matches_reference(tag):
    """oracle/rebuild.py against the reference's own _evict_to / PackedKVCache.rebuild
    (tests/golden/make_rebuild_golden.py): every written byte of the new storage, the
    lengths and the remapped slots of the live entries."""
    from oracle import rebuild as OR
    from tests._util import rebuild_case, same_bits

    c = rebuild_case(tag)
    new, lens, phys = OR.evict(c["in"], c["in_lens"], c["pos"], c["phys"], c["keep"],
                               next_position=c["next_position"], stage_mode=c["stage_mode"], mode=c["mode"],
                               repack_below=c["repack_below"], recent_window=c["recent_window"])
    assert lens == c["out_lens"]
    assert torch.equal(phys, c["out_phys"])
    for k, want in c["out"].items():
        assert same_bits(new[k], want), k


def test_rebuild_vectors_cover_padding():
    """The cases hold lanes with lists of different lengths, so the padding rules (a copy
    of old group 0 for a padded kept group, zeros for padded encoded / staged entries)
    are pinned by the vectors too."""
    from oracle import rebuild as OR
    from tests._util import rebuild_case

    pads = [0, 0, 0, 0]
    for tag in ("lazy", "lazy2", "full", "stage", "tail"):
        c = rebuild_case(tag)
        pos, phys = c["pos"].gather(-1, c["keep"]), c["phys"].gather(-1, c["keep"])
        lens = c["in_lens"]
        lists = OR.plan(phys, pos, lens, tail=lens[0] + lens[3] - c["next_position"], stage_mode=c["stage_mode"],
                        mode=c["mode"], repack_below=c["repack_below"], recent_window=c["recent_window"])
        for i, t in enumerate(lists):
            pads[i] += int((t < 0).sum())
    assert pads[0] > 0 and pads[1] > 0, pads
