"""In-tree build of the HIP library and the render_clean module (make + hipcc)."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def build(arch: str = "gfx950", jobs: int = 8) -> None:
    csrc = os.path.join(HERE, "csrc")
    # always recompile: the build check must see the current sources
    subprocess.run(["make", "-s", "-C", csrc, "clean"], check=True)
    subprocess.run(["make", "-s", "-C", csrc, f"-j{min(jobs, 16)}", f"ARCH={arch}", "all"],
                   check=True)
