"""Build libaspire_hip.so for gfx950 in-tree (hipcc, no cmake).

    python aspire_amd/csrc/build.py [--jobs N]

Objects go to aspire_amd/csrc/_build/, the library to aspire_amd/libaspire_hip.so.
Every source is recompiled on each call (the build check must exercise the
compiler); compiles run in parallel.
"""

from __future__ import annotations

import argparse
import hashlib
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
LIB = PKG / "libaspire_hip.so"
BUILD = HERE / "_build"
SOURCES = ["capi.cpp", "plan.cpp", "host_plan.cpp", "append.hip", "page_list.hip", "attention.hip", "select.hip",
           "rope_append.hip", "decode_ops.hip", "sampling.hip", "prefill.hip",
           "bandwidth.hip"]
ARCH = "gfx950"

COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function"]
# Packed fp32 VALU forms are disabled for all device code.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-munsafe-fp-atomics"]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    return str(path) if path.exists() else "hipcc"


def source_digest() -> str:
    h = hashlib.sha256()
    for name in sorted(SOURCES + ["common.h"]):
        h.update(name.encode())
        h.update((HERE / name).read_bytes())
    h.update((PKG.parent / "include" / "aspire_hip.h").read_bytes())
    return h.hexdigest()


# Per-source flags. prefill.hip: IEEE mode off, so fp32 max needs no NaN-quieting
# canonicalisation of MFMA results (its scores are never NaN once masked). Device
# compilation only: the host code's argument checks must still see NaN.
FILE_FLAGS = {"prefill.hip": ["-Xarch_device", "-mno-amdgpu-ieee", "-Xarch_device", "-fno-honor-nans"]}


def compile_one(src: str, defines: list[str], build_dir: Path = BUILD) -> Path:
    obj = build_dir / (src + ".o")
    cmd = [hipcc(), *COMMON, *FILE_FLAGS.get(src, []), *defines, "-c", str(HERE / src), "-o", str(obj)]
    if src.endswith(".hip"):
        cmd[1:1] = ["-x", "hip", *DEVICE]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{err}")
    if err.strip():
        print(f"[build] {src}:\n{err}", file=sys.stderr)
    return obj


def build(jobs: int | None = None, extra_defines: list[str] | None = None, out: Path | None = None) -> Path:
    """Compile every source and link the library (``out``, default the in-tree library).
    ``extra_defines`` (``NAME=VALUE``) select compile-time variants of the kernels, e.g.
    ``ASPIRE_DRAFT_VALU=1``; such a build goes to its own ``out`` and its objects to their
    own folder, so the default library is untouched."""
    extra = [f"-D{d}" for d in (extra_defines or [])]
    lib = Path(out) if out is not None else LIB
    build_dir = BUILD if not extra else BUILD / ("variant_" + hashlib.sha256(" ".join(extra).encode()).hexdigest()[:12])
    build_dir.mkdir(parents=True, exist_ok=True)
    digest = source_digest()
    flags = " ".join(COMMON + DEVICE + extra).replace('"', "")
    defines = [f'-DASPIRE_SOURCE_SHA256="{digest}"', f'-DASPIRE_BUILD_FLAGS="{flags}"', *extra]
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: compile_one(s, defines, build_dir), SOURCES))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, lib)
    return lib


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--define", action="append", default=[],
                    help="NAME=VALUE compile-time variant (repeatable); needs --out")
    ap.add_argument("--out", type=Path, default=None, help="library path for a variant build")
    args = ap.parse_args()
    if args.define and args.out is None:
        ap.error("a variant build (--define) needs its own --out library path")
    print(build(args.jobs, args.define, args.out))


if __name__ == "__main__":
    main()
