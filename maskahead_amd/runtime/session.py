"""Session-level operations of the read/keep path (the reference's
``maskahead.runtime.session``).

``value_score`` is the one scoring rule behind both decisions of the reference: the
selector feeds it the current block's mass, lookahead eviction the mass of the next
blocks (runtime/session.py:27-40).  Here it runs in the gfx950 kernels of
``ma_value_score``, with the reference's bf16 rounding points.
"""

from __future__ import annotations

import torch

from ..kernels.keep import value_score as _value_score


def value_score(a: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """a_i * ||v_i - c||, c = sum_j a_j v_j / sum_j a_j.  a [..., n] f32, v [..., n, d]
    -> [..., n] f32 (session.py:27-40).  The environment variable BITSIEVE_VSCORE_FP32=1
    selects the f32 branch, as in the reference."""
    return _value_score(a, v)
