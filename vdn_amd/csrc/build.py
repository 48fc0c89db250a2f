"""Builds libvdnmi.so (every HIP source in this directory) for gfx950 with hipcc.

Objects go to csrc/_build/, the shared library to vdn_amd/libvdnmi.so. Every call
recompiles (the build is the "does it build" check); sources compile in parallel.
"""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

CSRC = pathlib.Path(__file__).resolve().parent
PACKAGE = CSRC.parent
LIBRARY = PACKAGE / "libvdnmi.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    # Packed fp32 VALU ops are disabled for every kernel (they are not used on purpose and
    # some of their forms are not trusted on the target boxes).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libvdnmi")
    return path


def sources() -> list[pathlib.Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: pathlib.Path, out_dir: pathlib.Path) -> pathlib.Path:
    obj = out_dir / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = ("packed-fp32-ops", "is not a recognized feature")
    lines = [l for l in proc.stdout.splitlines() if not any(n in l for n in noise)]
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n" + "\n".join(lines))
    if any("warning" in l for l in lines):
        print("\n".join(lines), file=sys.stderr)
    return obj


def build(verbose: bool = False) -> pathlib.Path:
    out_dir = CSRC / "_build"
    out_dir.mkdir(exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), os.cpu_count() or 4, 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(lambda s: _compile(s, out_dir), srcs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError("hipcc link failed:\n" + proc.stdout)
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
