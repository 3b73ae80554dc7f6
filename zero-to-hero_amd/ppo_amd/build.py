"""Build libppo_amd.so for gfx950 in-tree (python -m ppo_amd.build)."""

from __future__ import annotations

import os
import subprocess

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "csrc")


def build(force: bool = True) -> str:
    """Compile every HIP source with hipcc (see csrc/Makefile); returns the
    path of the library.  `force` rebuilds even when the .so is up to date."""
    cmd = ["make", "-s", "-j8", "-C", CSRC]
    if force:
        cmd.insert(2, "-B")
    subprocess.run(cmd, check=True)
    from ._lib import LIB_PATH

    return LIB_PATH


if __name__ == "__main__":
    print(build())
