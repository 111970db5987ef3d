"""Builds libmnn.so (HIP kernels + C++ runtime + C ABI) for gfx950, in-tree.

Usage: python -m metalaudio_amd.build [--jobs N] [--debug] [--incremental]

The library lands in metalaudio_amd/lib/libmnn.so; every source is compiled by hipcc with
--offload-arch=gfx950 and packed-fp32 instruction selection disabled.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIB = PKG / "lib" / "libmnn.so"

ARCH = "gfx950"
COMMON_FLAGS = [
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libmnn.so")


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path, opt: list[str]) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *opt, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{msgs}")
    if msgs.strip():
        print(msgs, file=sys.stderr)
    return obj


def _stale(src: Path) -> bool:
    obj = BUILD / (src.name + ".o")
    if not obj.exists():
        return True
    deps = [src, *CSRC.glob("*.hpp"), *INCLUDE.glob("*.h")]
    return max(d.stat().st_mtime for d in deps) > obj.stat().st_mtime


def build(jobs: int | None = None, debug: bool = False, verbose: bool = True,
          incremental: bool = False) -> Path:
    """Compiles every source (or, with incremental, those older than a source or header) and
    links libmnn.so."""
    BUILD.mkdir(parents=True, exist_ok=True)
    LIB.parent.mkdir(parents=True, exist_ok=True)
    opt = ["-O0", "-g"] if debug else ["-O3"]
    srcs = sources()
    todo = [s for s in srcs if _stale(s)] if incremental else srcs
    jobs = jobs or min(max(len(todo), 1), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda s: _compile(s, opt), todo))
    objs = [BUILD / (s.name + ".o") for s in srcs]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB.relative_to(ROOT)} from {len(srcs)} sources")
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--debug", action="store_true")
    ap.add_argument("--incremental", action="store_true",
                    help="recompile only sources older than a source or header")
    args = ap.parse_args()
    build(args.jobs, args.debug, incremental=args.incremental)


if __name__ == "__main__":
    main()
