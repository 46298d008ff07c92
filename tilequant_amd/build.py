"""In-tree build of ``_lib/libtilequant_hip.so`` for gfx950.

``build()`` always recompiles what changed (make), so calling it after editing
a kernel source is enough; ``force=True`` rebuilds everything.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

CSRC = Path(__file__).resolve().parent / "csrc"


def build(force: bool = False, jobs: int = 8) -> Path:
    env = dict(os.environ)
    env.setdefault("HIPCC", "/opt/rocm/bin/hipcc")
    if force:
        subprocess.run(["make", "-s", "-C", str(CSRC), "clean"], check=True, env=env)
    subprocess.run(["make", "-s", f"-j{int(jobs)}", "-C", str(CSRC)], check=True, env=env)
    from ._native import LIB_PATH

    return LIB_PATH


if __name__ == "__main__":
    print(build(force=True))
