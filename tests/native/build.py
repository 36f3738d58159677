"""Build the native test programs under tests/native/_build/.

* tilemix_native runs the API validation table, the closed forms and every
  dense and routed GPU case through the HIP library's C++ API
  (include/attention_fused.h), with the C oracle linked as its checker; build
  the library first (tilemix-cuda_amd/build.py).
* quant_division_check runs the quantizer's division-free quotient against
  IEEE division for every fp16 (block maximum, value) pair, compiled with the
  library's own device flags.

Usage: python tests/native/build.py
"""
from __future__ import annotations

import importlib.util
import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
OUT = HERE / "_build"
EXE = OUT / "tilemix_native"
DIVISION_CHECK = OUT / "quant_division_check"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{result.stderr}{result.stdout}")


def build() -> Path:
    OUT.mkdir(parents=True, exist_ok=True)
    oracle_obj = OUT / "tilemix_oracle.o"
    _run(["gcc", "-O2", "-std=c99", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
          "-c", str(ROOT / "oracle" / "tilemix_oracle.c"), "-o", str(oracle_obj)])
    test_obj = OUT / "tilemix_native.o"
    _run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", f"-I{ROOT / 'include'}", f"-I{ROOT / 'oracle'}",
          "-Wno-unused-command-line-argument", "-c", str(HERE / "tilemix_native.cpp"), "-o", str(test_obj)])
    tmp = EXE.with_suffix(".tmp")
    _run([HIPCC, "--offload-arch=gfx950", str(test_obj), str(oracle_obj), "-fopenmp",
          f"-L{ROOT / 'tilemix-cuda_amd'}", "-ltilemix_hip", "-Wl,-rpath,$ORIGIN/../../../tilemix-cuda_amd",
          "-o", str(tmp)])
    os.replace(tmp, EXE)
    build_division_check()
    return EXE


def _library_build():
    spec = importlib.util.spec_from_file_location("tilemix_build", ROOT / "tilemix-cuda_amd" / "build.py")
    library_build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(library_build)
    return library_build


def build_division_check() -> Path:
    library_build = _library_build()
    OUT.mkdir(parents=True, exist_ok=True)
    tmp = DIVISION_CHECK.with_suffix(".tmp")
    _run([HIPCC, *[f for f in library_build.DEVICE_FLAGS if f != "-fPIC"], f"-I{ROOT / 'include'}",
          f"-I{library_build.CSRC}", str(HERE / "quant_division_check.hip"), "-o", str(tmp)])
    os.replace(tmp, DIVISION_CHECK)
    return DIVISION_CHECK


if __name__ == "__main__":
    print(f"built {build()}")
