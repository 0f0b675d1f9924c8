"""Build the gfx950 library in-tree: ninfer_amd/libninfer_amd.so.

Every HIP and C++ source under ninfer_amd/csrc is compiled by hipcc for gfx950 only, with packed
FP32 instructions disabled, then linked into one shared library exporting the C ABI declared in
include/ninfer_amd.h and include/ninfer_amd_runtime.h. Objects go to _build/ (git-ignored); the
.so stays next to this file so it travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "ninfer_amd" / "csrc"
BUILD = ROOT / "_build" / "ninfer_amd"
OUT = ROOT / "ninfer_amd" / "libninfer_amd.so"
ARCH = "gfx950"

COMMON = [
    "-O3",
    "-std=c++20",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-fast-math",
    "-Wall",
    "-Wno-unused-function",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return hipcc


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [_hipcc(), *COMMON, *lang, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    sources = sorted(p for p in CSRC.iterdir() if p.suffix in (".hip", ".cpp"))
    jobs = min(8, os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT.relative_to(ROOT)} from {len(sources)} sources")
    return OUT


if __name__ == "__main__":
    build()
