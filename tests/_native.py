"""Build helper for the tests' own HIP code (test infrastructure, not the
operator library): tests/f8_encoder_check.hip -> tests/libf8check.so.

    python tests/_native.py        # build it ahead of a GPU run

The GPU test that uses the library builds it here first if it is missing, so
a fresh checkout still runs; building ahead keeps compilation out of GPU runs.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "f8_encoder_check.hip"
LIB = HERE / "libf8check.so"

sys.path.insert(0, str(HERE.parent))
from muxi_race_amd.build import HIP_FLAGS, _hipcc  # noqa: E402


def build_f8check(force: bool = False) -> Path:
    """Compile the fp8 encoder check into tests/libf8check.so (skipped when it
    is newer than its sources, unless ``force``); returns its path."""
    deps = [SRC, HERE.parent / "muxi_race_amd" / "csrc" / "moe_common.h"]
    if not force and LIB.exists() and LIB.stat().st_mtime >= max(d.stat().st_mtime for d in deps):
        return LIB
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), *HIP_FLAGS, "-shared", str(SRC), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {SRC.name}:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build_f8check(force=True))
