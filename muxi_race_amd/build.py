"""Build libmoe_gfx950.so in-tree with hipcc (gfx950 only).

    python -m muxi_race_amd.build          # or muxi_race_amd.build.build()

Each .hip source under csrc/ is compiled to an object in parallel, then linked
into ``muxi_race_amd/libmoe_gfx950.so`` next to this file.  The packed-fp32
target feature is switched off for device code (see ``HIP_FLAGS``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJDIR = PKG / "_build"
LIB = PKG / "libmoe_gfx950.so"
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # no packed-fp32 VALU ops in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (need ROCm with gfx950 support)")


def _compile(src: Path, obj: Path, extra=()) -> tuple[Path, str]:
    cmd = [_hipcc(), *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(
        ln for ln in (r.stdout + r.stderr).splitlines()
        if "packed-fp32-ops" not in ln  # host pass does not know the feature
    )
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{msgs}")
    return obj, msgs


def build(verbose: bool = False, defines: dict | None = None, out: Path | None = None) -> Path:
    """Compile every csrc/*.hip and link the shared library; returns its path.

    ``defines`` adds -DNAME=VALUE tuning macros (e.g. MOE_S2_STAGES_128) and
    ``out`` redirects the library (default: muxi_race_amd/libmoe_gfx950.so)."""
    lib = LIB if out is None else Path(out)
    objdir = OBJDIR if out is None else lib.parent / "_build"
    objdir.mkdir(parents=True, exist_ok=True)
    extra = [f"-D{k}={v}" for k, v in (defines or {}).items()]
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_compile, s, objdir / (s.stem + ".o"), extra) for s in srcs]
        objs = []
        for f in futs:
            obj, msgs = f.result()
            objs.append(obj)
            if verbose and msgs.strip():
                print(msgs, file=sys.stderr)
    tmp = lib.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}{r.stderr}")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose=True))
