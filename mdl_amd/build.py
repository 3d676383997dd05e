"""Build libmdl_hip.so for gfx950 in-tree (``python -m mdl_amd.build``)."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent / "csrc"


def build(jobs: int | None = None, force: bool = True) -> Path:
    """Compile every HIP source with hipcc and link the shared library."""

    jobs = jobs or min(8, os.cpu_count() or 1)
    if force:
        subprocess.run(["make", "-C", str(CSRC), "clean"], check=True, stdout=subprocess.DEVNULL)
    subprocess.run(["make", "-C", str(CSRC), f"-j{jobs}"], check=True)
    out = CSRC.parent / "libmdl_hip.so"
    if not out.exists():
        raise RuntimeError("hipcc build finished without producing libmdl_hip.so")
    return out


if __name__ == "__main__":
    print(build(force="--incremental" not in sys.argv))
