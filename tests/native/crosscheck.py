"""JSONL fixture cross-check harness (test infrastructure).

Counterpart of the reference's python/reference_attention.py:27-82 for this
build: ``self_check`` validates the CPU PyTorch oracle
(oracle/torch_reference.py) against float64 and closed forms, and
``check_native`` runs the native test driver (tests/native/_build/tilemix_test,
the restatement of the reference's test binary) with ``--export-json FILE``,
then compares every exported dense case - one JSON object per line with keys
m, n, d, pattern, q, k, v (fp16 values), o (fp32 GPU output) - against
softmax(Q K^T / sqrt(d)) V computed in float64 on the CPU, at the reference's
tolerance (atol 1e-5, rtol 1e-4).

Usage: python tests/native/crosscheck.py [--native-test tests/native/_build/tilemix_test]
"""
from __future__ import annotations

import argparse
import json
import subprocess
import sys
import tempfile
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle.torch_reference import reference_attention  # noqa: E402

FIELDS = ("m", "n", "d", "pattern", "q", "k", "v", "o")


def _errors(actual: torch.Tensor, expected: torch.Tensor) -> str:
    error = (actual - expected).abs()
    relative = error / expected.abs().clamp_min(1e-5)
    return (f"max_abs_error={error.max().item():.9g} max_rel_error={relative.max().item():.9g} "
            f"rms_error={error.square().mean().sqrt().item():.9g}")


def self_check() -> None:
    """float32 CPU oracle vs float64 and closed forms (python/reference_attention.py:27-53)."""
    generator = torch.Generator(device="cpu").manual_seed(20261029)
    for m, n, d in ((1, 1, 1), (3, 5, 7), (17, 33, 17), (64, 64, 32)):
        q = torch.randn((m, d), generator=generator).half()
        k = torch.randn((n, d), generator=generator).half()
        v = torch.randn((n, d), generator=generator).half()
        actual = reference_attention(q, k, v)
        expected = reference_attention(q, k, v, compute_dtype=torch.float64)
        torch.testing.assert_close(actual.double(), expected, atol=1e-5, rtol=1e-4)
        print(f"PASS CPU PyTorch M={m} N={n} d={d} atol=1e-5 rtol=1e-4 {_errors(actual.double(), expected)}")
    q = torch.zeros((3, 7), dtype=torch.float16)
    k = torch.ones((5, 7), dtype=torch.float16)
    v = torch.arange(35, dtype=torch.float16).reshape(5, 7)
    torch.testing.assert_close(reference_attention(q, k, v), v.float().mean(0).expand(3, 7))
    torch.testing.assert_close(reference_attention(q, k[:1], v[:1]), v[:1].float().expand(3, 7))
    q = torch.tensor([[1000.0]], dtype=torch.float16)
    k = torch.tensor([[1000.0], [-1000.0]], dtype=torch.float16)
    v = torch.tensor([[3.0], [-7.0]], dtype=torch.float16)
    torch.testing.assert_close(reference_attention(q, k, v), torch.tensor([[3.0]]))
    print("PASS CPU PyTorch uniform, single-key, and extreme-logit checks")


def check_fixtures(path: Path) -> int:
    """Compare every fixture of a JSONL file; returns the number checked."""
    count = 0
    with path.open() as source:
        for line_number, line in enumerate(source, 1):
            case = json.loads(line)
            missing = [key for key in FIELDS if key not in case]
            if missing:
                raise ValueError(f"{path}:{line_number}: fixture lacks {missing}")
            m, n, d = case["m"], case["n"], case["d"]
            q = torch.tensor(case["q"], dtype=torch.float16).reshape(m, d)
            k = torch.tensor(case["k"], dtype=torch.float16).reshape(n, d)
            v = torch.tensor(case["v"], dtype=torch.float16).reshape(n, d)
            actual = torch.tensor(case["o"], dtype=torch.float32).reshape(m, d).double()
            expected = reference_attention(q, k, v, compute_dtype=torch.float64)
            torch.testing.assert_close(actual, expected, atol=1e-5, rtol=1e-4)
            print(f"PASS GPU vs CPU PyTorch FP64 M={m} N={n} d={d} pattern={case['pattern']} "
                  f"atol=1e-5 rtol=1e-4 {_errors(actual, expected)}")
            count += 1
    return count


def check_native(executable: Path) -> int:
    """Run the native suite with --export-json, then cross-check its fixtures."""
    with tempfile.TemporaryDirectory(prefix="tilemix-fixtures-") as directory:
        fixtures = Path(directory) / "attention.jsonl"
        subprocess.run([str(Path(executable).resolve()), "--export-json", str(fixtures)], check=True)
        count = check_fixtures(fixtures)
    if count == 0:
        raise RuntimeError("the native suite exported no fixtures")
    print(f"PASS {count} GPU fixtures agree with the independent CPU PyTorch oracle")
    return count


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--native-test", type=Path, help="path to the built tests/native/_build/tilemix_test")
    args = parser.parse_args()
    torch.set_num_threads(1)
    with torch.inference_mode():
        print(f"PyTorch={torch.__version__} HIP={torch.version.hip} oracle_device=CPU")
        self_check()
        if args.native_test:
            check_native(args.native_test)
    return 0


if __name__ == "__main__":
    sys.exit(main())
