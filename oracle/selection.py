"""Selection helpers of the CPU oracle -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Thin torch front ends over oracle/codec.c plus the boundary-tolerance comparison the
parity tests use for index sets computed from floating-point scores.
"""

from __future__ import annotations

import numpy as np
import torch

from . import codec


def topk_ascending(rank: torch.Tensor, k: int, mask: torch.Tensor | None = None) -> torch.Tensor:
    """Read set of session.py:1429-1438 with index-ascending tie-break (oracle/codec.c)."""
    m = None if mask is None else mask.to(torch.uint8).cpu().numpy()
    return torch.from_numpy(codec.topk_ascending(rank.float().cpu().numpy(), k, m))


def keep_select(pos: torch.Tensor, score: torch.Tensor, capacity: int, window: int,
                sink_tokens: int = 0, pin=None) -> torch.Tensor:
    """Keep set of eviction.py:355-409 (oracle/codec.c)."""
    return torch.from_numpy(codec.keep_select(pos.cpu().numpy(), score.float().cpu().numpy(),
                                              capacity, window, sink_tokens, pin))


def boundary_mismatch_ok(got: torch.Tensor, want: torch.Tensor, score: torch.Tensor,
                         k: int, rel: float, mask: torch.Tensor | None = None):
    """Compare two index sets selected by top-k from (nearly) the same scores.

    got, want [..., k] index sets; score [..., n] the oracle's scores.  Every index in
    one set and not the other must have an oracle score within `rel` (relative) of the
    k-th largest live oracle score of its row: those are the ties / near-ties at the
    selection boundary that float summation order may resolve either way.
    Returns (ok, n_mismatched, worst_relative_distance)."""
    got = got.reshape(-1, got.shape[-1]).cpu().numpy()
    want = want.reshape(-1, want.shape[-1]).cpu().numpy()
    sc = score.reshape(-1, score.shape[-1]).double().cpu().numpy()
    mk = None if mask is None else mask.reshape(-1, mask.shape[-1]).bool().cpu().numpy()
    worst, nmis = 0.0, 0
    for r in range(got.shape[0]):
        s = sc[r].copy()
        if mk is not None:
            s[~mk[r]] = -np.inf
        kth = np.sort(s)[::-1][k - 1]
        diff = set(got[r].tolist()) ^ set(want[r].tolist())
        nmis += len(diff)
        for j in diff:
            d = abs(s[j] - kth) / max(abs(kth), 1e-30)
            worst = max(worst, d)
    return worst <= rel, nmis, worst
