"""Build libfq_hip.so in-tree for gfx950 (hipcc via flashquest_amd/csrc/Makefile)."""
from __future__ import annotations

import os
import subprocess
import sys

CSRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc")


def build(jobs: int = 8, force: bool = False) -> str:
    if force:
        subprocess.run(["make", "-C", CSRC, "clean"], check=True, stdout=subprocess.DEVNULL)
    subprocess.run(["make", "-C", CSRC, f"-j{min(jobs, 16)}"], check=True)
    return os.path.join(os.path.dirname(CSRC), "_lib", "libfq_hip.so")


if __name__ == "__main__":
    print(build(force="--force" in sys.argv))
