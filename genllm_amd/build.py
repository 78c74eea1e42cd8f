"""Build step for libgenllm_hip.so (gfx950) -- see genllm_amd/csrc/Makefile."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libgenllm_hip.so")


def build_library(clean: bool = True, jobs: int = 8) -> str:
    """Compile every HIP source for gfx950 and link libgenllm_hip.so."""
    if clean:
        subprocess.run(["make", "-s", "-C", CSRC, "clean"], check=True)
    subprocess.run(["make", "-s", "-C", CSRC, f"-j{jobs}"], check=True)
    if not os.path.exists(LIB):
        raise RuntimeError("build did not produce " + LIB)
    return LIB
