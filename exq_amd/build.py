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

SOURCES = ["elementwise.hip", "routing.hip", "pack.hip", "moe_mfma.hip", "decode.hip", "prefill.hip", "general.hip", "noalloc.hip"]

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
    # per-kernel register / scratch report, checked below
    "-Rpass-analysis=kernel-resource-usage",
]


def _resource_report(text: str) -> dict:
    """{kernel: {"scratch": bytes/lane, "vgprs": n, "agprs": n, "occupancy": waves/SIMD}}"""
    out, cur = {}, None
    for line in text.splitlines():
        if "remark:" not in line:
            continue
        body = line.split("remark:", 1)[1].strip()
        body = body.replace("[-Rpass-analysis=kernel-resource-usage]", "").strip()
        if body.startswith("Function Name:"):
            cur = body.split(":", 1)[1].strip()
            out[cur] = {}
        elif cur is not None and ":" in body:
            key, val = body.rsplit(":", 1)
            key = key.strip()
            val = val.strip()
            if key.startswith("ScratchSize"):
                out[cur]["scratch"] = int(val)
            elif key == "VGPRs":
                out[cur]["vgprs"] = int(val)
            elif key == "AGPRs":
                out[cur]["agprs"] = int(val)
            elif key.startswith("Occupancy"):
                out[cur]["occupancy"] = int(val)
    return out


def _compile(src: Path, obj: Path) -> str:
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    text = r.stdout + r.stderr
    err = "\n".join(l for l in text.splitlines()
                    if noise not in l and "kernel-resource-usage" not in l
                    and not l.lstrip().startswith(("|", "^")) and not l[:6].strip().isdigit())
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    # A kernel that spills to scratch streams its spills through HBM: refuse it.
    spilled = {k: v for k, v in _resource_report(text).items() if v.get("scratch", 0) > 0}
    if spilled:
        raise RuntimeError(f"{src.name}: kernels use scratch memory: {spilled}")
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
