"""Builds libperegrine_hip.so in-tree (hipcc --offload-arch=gfx950)."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")


def build(jobs: int = 4) -> str:
    """Compile every HIP source; always rebuilds. Returns the library path."""
    subprocess.run(["make", "-s", "-B", f"-j{jobs}", "-C", CSRC], check=True)
    return os.path.join(HERE, "libperegrine_hip.so")


if __name__ == "__main__":
    print(build())
