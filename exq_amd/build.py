"""Build libexq_hip.so (gfx950) from exq_amd/csrc with hipcc.

Usage: ``python -m exq_amd.build`` (or ``__graft_entry__.build()``).
Objects go to ``exq_amd/_build/``; the library to ``exq_amd/libexq_hip.so``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libexq_hip.so"

SOURCES = ["elementwise.hip", "routing.hip", "pack.hip", "moe_mfma.hip", "decode.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Keep the compiler away from packed-FP32 VALU forms.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _compile(src: Path, obj: Path) -> str:
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    return err


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the shared library."""
    BUILD.mkdir(exist_ok=True)
    jobs = []
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        for s in SOURCES:
            src = CSRC / s
            obj = BUILD / (src.stem + ".o")
            jobs.append((s, ex.submit(_compile, src, obj)))
        for s, fut in jobs:
            msg = fut.result()
            if verbose and msg.strip():
                print(f"[{s}]\n{msg}")
    objs = [str(BUILD / (Path(s).stem + ".o")) for s in SOURCES]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv or True)
