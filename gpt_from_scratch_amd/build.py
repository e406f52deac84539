"""Build libmi_attn.so in-tree with hipcc (gfx950) through csrc/Makefile."""
from __future__ import annotations

import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(_HERE, "csrc")


def build_library(force: bool = True, jobs: int = 8) -> str:
    """Compile every HIP source and link libmi_attn.so; returns its path."""
    cmd = ["make", "-C", CSRC, f"-j{jobs}"]
    if force:
        cmd.insert(1, "-B")
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building libmi_attn.so failed:\n{res.stdout[-8000:]}")
    return os.path.join(_HERE, "libmi_attn.so")


if __name__ == "__main__":
    print(build_library())
