"""Build recipe for libakasha_hip.so (gfx950) and the CPU oracle.

``build_library()`` always recompiles (make -B) so a call is a real "does it
build" check; ``build_oracle()`` compiles oracle/liboracle.so, the test-only
CPU checker (the product library never links it).
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent


def _run(cmd, cwd):
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build failed in {cwd}: {' '.join(cmd)}\n{r.stdout[-8000:]}")
    return r.stdout


def build_library(force: bool = True) -> Path:
    jobs = str(min(16, os.cpu_count() or 4))
    cmd = ["make", "-j", jobs] + (["-B"] if force else [])
    _run(cmd, PKG / "csrc")
    lib = PKG / "libakasha_hip.so"
    if not lib.exists():
        raise RuntimeError("libakasha_hip.so was not produced")
    return lib


def build_oracle(force: bool = True) -> Path:
    cmd = ["make"] + (["-B"] if force else [])
    _run(cmd, ROOT / "oracle")
    return ROOT / "oracle" / "liboracle.so"


if __name__ == "__main__":
    print(build_library())
    print(build_oracle())
