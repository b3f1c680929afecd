"""Write the golden vectors that only the reference itself can pin.

Run in the build container (where /root/reference exists):

    python tests/golden/make_golden.py

It imports the reference package (brain-lab-research/MaskAhead, src/maskahead) and
evaluates, on small seeded CPU inputs, the two functions whose exact rounding no closed
form fixes:

  * value_score (runtime/session.py:27-40), the keep-path score computed in bf16;
  * quantize_keys / quantize_values (reference.py:58-90, 182-213) fed bf16 input, whose
    min / range / division / round-half-even run in bf16 arithmetic.

Only inputs and outputs are written (golden_vectors.npz); nothing of the reference is
copied.  The test suite (tests/test_oracle_golden.py) checks the CPU oracle against
these vectors, and the GPU tests check the HIP kernels against the oracle.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

REF = Path("/root/reference/src")
OUT = Path(__file__).resolve().parent / "golden_vectors.npz"


def _bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    sys.path.insert(0, str(REF))
    from maskahead.reference import quantize_keys, quantize_values   # noqa: E402
    from maskahead.runtime.session import value_score                # noqa: E402

    g = torch.Generator("cpu").manual_seed(1234)
    out: dict[str, np.ndarray] = {}

    # value_score: a [L=1, B=1, H=3, n] f32 (mass-like, some zeros), v bf16 [.., n, 128]
    for tag, n in (("vs_small", 40), ("vs_mid", 300)):
        a = torch.rand((1, 1, 3, n), generator=g) ** 3 / n
        a[..., ::7] = 0.0
        v = (torch.randn((1, 1, 3, n, 128), generator=g) * 1.5).to(torch.bfloat16)
        s = value_score(a, v)
        out[f"{tag}_a"] = a.numpy()
        out[f"{tag}_v"] = _bits16(v)
        out[f"{tag}_score"] = s.numpy()

    # quantizers fed bf16 and f32 input
    for dt, tag in ((torch.bfloat16, "bf16"), (torch.float32, "f32")):
        x = torch.randn((1, 2, 64, 128), generator=g) * torch.empty((1, 2, 1, 128)).log_normal_(0, 0.5, generator=g)
        x[:, :, :4] *= 8
        x[0, 0, 5, 3] = x[0, 0, 6, 3]            # a repeated value
        x[0, 1, 32:64, 7] = 0.25                 # a constant group (scale clamps to 1e-8)
        x = x.to(dt)
        pk = quantize_keys(x, bits=4, token_group=32, param_dtype=torch.float16)
        pv = quantize_values(x, bits=4, channel_group=32, param_dtype=torch.float16)
        out[f"q_{tag}_x"] = _bits16(x) if dt == torch.bfloat16 else x.numpy()
        out[f"q_{tag}_kq"] = pk.payload.numpy()
        out[f"q_{tag}_ks"] = _bits16(pk.scale)
        out[f"q_{tag}_kz"] = _bits16(pk.zero)
        out[f"q_{tag}_vq"] = pv.payload.numpy()
        out[f"q_{tag}_vs"] = _bits16(pv.scale)
        out[f"q_{tag}_vz"] = _bits16(pv.zero)

    np.savez(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
