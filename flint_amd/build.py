"""Build step of the HIP backend: compiles libthuban_hip.so for gfx950 in-tree."""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")


def build(jobs: int = 8, force: bool = True) -> str:
    """Runs the committed Makefile; returns the path of the built library."""
    args = ["make", "-C", CSRC, f"-j{jobs}"]
    if force:
        args.append("-B")
    subprocess.run(args, check=True)
    return os.path.join(HERE, "libthuban_hip.so")


if __name__ == "__main__":
    print(build())
