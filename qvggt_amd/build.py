"""Build libqvggt_hip.so in-tree with hipcc for gfx950.

    python -m qvggt_amd.build            # compile every csrc/*.hip, link the .so

Objects go to ``qvggt_amd/_build/``; the library to ``qvggt_amd/lib/``.  No
torch headers are involved: the library is a plain C ABI (include/qvggt_hip.h).
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
BUILD = PKG / "_build"
LIBDIR = PKG / "lib"
LIBNAME = "libqvggt_hip.so"
ARCH = os.environ.get("QVGGT_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC",
    # packed-fp32 VALU forms are kept out of generated code on purpose
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (need ROCm in /opt/rocm)")


def _compile(src: Path, obj: Path) -> tuple[Path, str]:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (p.stdout + p.stderr).splitlines() if noise not in l)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    return obj, err


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip (always, even if a library exists) and link."""
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    objs = []
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = {ex.submit(_compile, s, BUILD / (s.stem + ".o")): s for s in srcs}
        for f in cf.as_completed(futs):
            obj, warn = f.result()
            objs.append(obj)
            if verbose:
                print(f"[qvggt build] compiled {futs[f].name}", flush=True)
                if warn.strip():
                    print(warn, flush=True)
    out = LIBDIR / LIBNAME
    tmp = LIBDIR / (LIBNAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, sorted(objs))]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("link failed:\n" + p.stdout + p.stderr)
    os.replace(tmp, out)
    if verbose:
        print(f"[qvggt build] linked {out}", flush=True)
    return out


if __name__ == "__main__":
    build()
    sys.exit(0)
