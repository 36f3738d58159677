"""Exhaustive GPU pin of the quantizer's division-free quotient.

The quantizer (src/tilemix.cu:23-48 restated in tilemix_device.h) computes
round(x / scale) per element. The HIP kernels replace the division by the
block's reciprocal plus one exact correction step; tests/native/
quant_division_check.hip compares that with IEEE division on the device for
every positive finite fp16 block maximum and every fp16 value not above it
(about 1.0e9 pairs), as fp32 quotients and as int8 results, for each of the
per-element forms the kernels use (quantize_value_recip, quantize_in_block
and both lanes of quantize_half), and checks pack_bytes on every int8 value.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

CHECK = Path(__file__).resolve().parent / "native" / "_build" / "quant_division_check"


def test_division_free_quotient_is_exact(cuda):
    if not CHECK.exists():
        pytest.fail(f"{CHECK} is not built; run python tests/native/build.py")
    print("quant_division_check: all fp16 (absmax, x) pairs", flush=True)
    result = subprocess.run([str(CHECK)], capture_output=True, text=True, timeout=90)
    print(result.stdout, result.stderr, flush=True)
    assert result.returncode == 0, result.stdout + result.stderr
    assert result.stdout.startswith("PASS "), result.stdout
    # 1007713278 (absmax, x) pairs plus 256 pack_bytes values.
    assert int(result.stdout.split()[1]) == 1007713278 + 256
