"""Build step: compiles libqb_gdn.so (HIP for gfx950 plus the C ABI) in-tree with the Makefile beside this file."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def build(jobs: int = 8, force: bool = True) -> str:
    """Compiles every HIP source. force rebuilds from scratch, so a stale object never survives a source change."""
    if force:
        subprocess.run(["make", "-C", HERE, "-s", "clean"], check=True)
    subprocess.run(["make", "-C", HERE, "-s", f"-j{jobs}"], check=True)
    return os.path.join(HERE, "libqb_gdn.so")


if __name__ == "__main__":
    print(build())
