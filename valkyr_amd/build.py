"""In-tree build of libvkhip.so (hipcc --offload-arch=gfx950) via the csrc Makefile."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libvkhip.so")


def build_library(jobs: int = 8, force: bool = True) -> str:
    jobs = max(1, min(int(jobs), 16))
    if force:
        # always recompile: the build check must exercise the compiler
        subprocess.run(["make", "-s", "-C", CSRC, "clean"], check=True)
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", CSRC], check=True)
    if not os.path.exists(LIB):
        raise RuntimeError(f"build did not produce {LIB}")
    return LIB


if __name__ == "__main__":
    print(build_library())
