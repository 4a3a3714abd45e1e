"""Build libmoehip.so for gfx950 with hipcc (ffai_amd/csrc/Makefile)."""
from __future__ import annotations

import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(_HERE, "csrc")


def build(force: bool = True, jobs: int | None = None) -> str:
    """Compile every HIP translation unit for gfx950 and link the library.

    ``force`` rebuilds from scratch (the driver's build check wants a real
    compile every call)."""
    jobs = jobs or min(8, os.cpu_count() or 1)
    cmd = ["make", "-C", CSRC, f"-j{jobs}"]
    if force:
        cmd.append("-B")
    subprocess.run(cmd, check=True)
    return os.path.join(_HERE, "libmoehip.so")


if __name__ == "__main__":
    print(build())
