"""The oracle's selection rules (oracle/codec.c) pinned by brute force on tiny inputs
and by invariants: read-set top-k (session.py:1429-1438) and keep set
(eviction.py:325-409)."""

import math
import random

import numpy as np
import torch

from oracle import codec
from oracle import selection as OS


def _brute_topk(vals, k, live=None):
    """k largest (dead -> -inf, NaN above +inf), ties by index, returned ascending."""
    def rank(i):
        v = vals[i] if (live is None or live[i]) else -math.inf
        return math.inf if v != v else v
    order = sorted(range(len(vals)), key=lambda i: (-rank(i), i))
    return sorted(order[:k])


def test_topk_brute_force_with_ties():
    rng = random.Random(0)
    for trial in range(200):
        n = rng.randint(1, 40)
        vals = [float(rng.choice([0.0, 1.0, 2.0, 2.0, -1.0, rng.random()])) for _ in range(n)]
        live = [rng.random() > 0.2 for _ in range(n)]
        k = rng.randint(0, n)
        got = codec.topk_ascending(np.array([vals], np.float32), k, np.array([live], np.uint8))[0].tolist()
        assert got == _brute_topk(vals, k, live), (vals, live, k)


def test_topk_matches_torch_without_ties():
    g = torch.Generator().manual_seed(1)
    x = torch.rand((3, 500), generator=g)
    got = OS.topk_ascending(x, 37)
    want = x.topk(37).indices.sort().values
    assert torch.equal(got, want)


def test_topk_signed_zero_and_nan():
    x = np.array([[-0.0, 0.0, np.nan, 1.0, -np.inf]], np.float32)
    # NaN ranks first, then 1.0, then the two zeros by index
    assert codec.topk_ascending(x, 3).tolist() == [[0, 2, 3]]


def _brute_keep(pos, score, cap, w, sinks=0, pin=None):
    """eviction.py:355-409 read as a set definition."""
    n = len(pos)
    w = min(w, cap)
    recent = set(sorted(range(n), key=lambda i: -pos[i])[:w])
    def rank(i):
        if i in recent:
            return -math.inf
        r = score[i]
        if pos[i] < sinks or (pin and pin[0] <= pos[i] < pin[1]):
            r = math.inf
        return r
    rest = sorted((i for i in range(n)), key=lambda i: (-rank(i), i))[:cap - w]
    keep = list(recent) + rest
    return sorted(keep, key=lambda i: pos[i])


def test_keep_select_brute_force():
    rng = random.Random(2)
    for trial in range(200):
        n = rng.randint(2, 50)
        pos = rng.sample(range(200), n)
        score = [rng.choice([0.0, 0.5, rng.random()]) for _ in range(n)]
        cap = rng.randint(1, n)
        w = rng.randint(0, cap + 3)
        sinks = rng.choice([0, 4, 20])
        pin = rng.choice([None, (30, 60)])
        got = codec.keep_select(np.array([pos]), np.array([score], np.float32), cap, w, sinks, pin)[0].tolist()
        assert got == _brute_keep(pos, score, cap, w, sinks, pin), (pos, score, cap, w, sinks, pin)


def test_keep_select_invariants():
    g = torch.Generator().manual_seed(3)
    n, cap, w, sinks = 1000, 200, 64, 4
    pos = torch.arange(n).expand(2, 3, n).contiguous()
    score = torch.rand((2, 3, n), generator=g)
    keep = OS.keep_select(pos, score, cap, w, sinks)
    assert keep.shape == (2, 3, cap)
    kp = torch.gather(pos, -1, keep)
    assert torch.all(kp[..., 1:] > kp[..., :-1])                   # ordered by position
    assert torch.all((kp >= n - w).sum(-1) == w)                  # the W newest
    assert torch.all((kp < sinks).sum(-1) == sinks)               # every sink


def test_compact_rows():
    rng = np.random.default_rng(4)
    src = rng.integers(0, 255, size=(2, 50, 8), dtype=np.uint8)
    keep = np.sort(rng.choice(50, size=(2, 20), replace=True), axis=-1)
    got = codec.compact_rows(src, keep)
    want = np.take_along_axis(src, keep[..., None].repeat(8, -1), axis=1)
    assert np.array_equal(got, want)
