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
