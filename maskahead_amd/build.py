"""Build libmaskahead_hip.so in-tree with hipcc for gfx950 (make, maskahead_amd/csrc/Makefile)."""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

CSRC = Path(__file__).resolve().parent / "csrc"


def build(jobs: int | None = None, force: bool = False) -> Path:
    """Compile every HIP source; returns the library path.  force=True rebuilds all."""
    jobs = jobs or min(8, os.cpu_count() or 1)
    if force:
        subprocess.run(["make", "-s", "-C", str(CSRC), "clean"], check=True)
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", str(CSRC)], check=True)
    return CSRC.parent / "libmaskahead_hip.so"


if __name__ == "__main__":
    print(build())
