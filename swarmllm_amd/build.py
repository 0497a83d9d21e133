"""Builds libqmm.so in-tree from swarmllm_amd/csrc (hipcc, gfx950)."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")


def build_library(jobs: int = 4, force: bool = True) -> str:
    if force:
        subprocess.run(["make", "-s", "-C", CSRC, "clean"], check=True)
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", CSRC], check=True)
    out = os.path.join(HERE, "libqmm.so")
    if not os.path.exists(out):
        raise RuntimeError("libqmm.so was not produced")
    # the M0 invariant of csrc/lds_copy.h over the AMD assembly just built
    from .m0_check import check_build

    check_build(os.path.join(CSRC, "_build"))
    return out
