"""Build the gfx950 TileMix library and its demo driver with hipcc.

Outputs (in-tree, git-ignored, shipped with the tree to the GPU host):
  tilemix-cuda_amd/libtilemix_hip.so        the library (C ABI of include/tilemix_capi.h)
  tilemix-cuda_amd/_build/tilemix_demo      demo driver (restates the reference src/main.cu)

Usage: python tilemix-cuda_amd/build.py [--lib-only] [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = ROOT / "include"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libtilemix_hip.so"
DEMO = BUILD / "tilemix_demo"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Device flags: correctly rounded binary32 division (the quantizer's
# reciprocal 1/scale must be the IEEE one for its quotients to equal x/scale),
# and no packed-FP32 VALU instructions (v_pk_*_f32) in generated code.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-fast-math",
    "-ffp-contract=fast",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]

LIB_SOURCES = ["quantize.hip", "attention.hip", "routing.hip"]
SOURCE_FLAGS: dict[str, list[str]] = {}


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature flag; that
    # warning is expected and filtered.
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{err}\n{result.stdout}")
    if err.strip():
        print(err, file=sys.stderr)


def compile_object(source: Path, obj: Path) -> Path:
    obj.parent.mkdir(parents=True, exist_ok=True)
    _run([HIPCC, *DEVICE_FLAGS, *SOURCE_FLAGS.get(source.name, []), f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(source),
          "-o", str(obj)])
    return obj


def build_library(jobs: int) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    with futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(lambda s: compile_object(CSRC / s, BUILD / (s + ".o")), LIB_SOURCES))
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)])
    os.replace(tmp, LIBRARY)
    return LIBRARY


def build_demo() -> Path:
    obj = BUILD / "demo_main.o"
    _run([HIPCC, f"--offload-arch={ARCH}", "-O2", "-std=c++17", f"-I{INCLUDE}",
          "-Wno-unused-command-line-argument", "-c", str(PACKAGE / "examples" / "demo_main.cpp"), "-o", str(obj)])
    tmp = DEMO.with_suffix(".tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", str(obj), f"-L{PACKAGE}", "-ltilemix_hip",
          "-Wl,-rpath,$ORIGIN/..", "-o", str(tmp)])
    os.replace(tmp, DEMO)
    return DEMO


def build_all(lib_only: bool = False, jobs: int | None = None) -> None:
    jobs = jobs or min(8, os.cpu_count() or 1)
    build_library(jobs)
    if lib_only:
        return
    build_demo()


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--lib-only", action="store_true")
    parser.add_argument("--jobs", type=int, default=None)
    args = parser.parse_args()
    build_all(lib_only=args.lib_only, jobs=args.jobs)
    print(f"built {LIBRARY}")


if __name__ == "__main__":
    main()
