"""The JSONL fixture cross-check harness (tests/native/crosscheck.py): its CPU
self-check and fixture parser without a GPU; the full native export and
cross-check on the GPU."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "native"))
import crosscheck  # noqa: E402

NATIVE = HERE / "native" / "_build" / "tilemix_test"


def test_self_check_passes():
    with torch.inference_mode():
        crosscheck.self_check()


def _write(path, cases):
    with path.open("w") as f:
        for c in cases:
            f.write(json.dumps(c) + "\n")


def test_fixture_check_accepts_exact_and_rejects_wrong(tmp_path):
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(s, generator=g).half() for s in ((4, 8), (6, 8), (6, 8)))
    o = crosscheck.reference_attention(q, k, v, compute_dtype=torch.float64).float()
    case = {"m": 4, "n": 6, "d": 8, "pattern": "random", "q": q.flatten().tolist(), "k": k.flatten().tolist(),
            "v": v.flatten().tolist(), "o": o.flatten().tolist()}
    good = tmp_path / "good.jsonl"
    _write(good, [case, case])
    assert crosscheck.check_fixtures(good) == 2
    bad = dict(case, o=(o + 1e-3).flatten().tolist())
    path = tmp_path / "bad.jsonl"
    _write(path, [case, bad])
    with pytest.raises(AssertionError):
        crosscheck.check_fixtures(path)
    incomplete = {key: value for key, value in case.items() if key != "o"}
    path = tmp_path / "incomplete.jsonl"
    _write(path, [incomplete])
    with pytest.raises(ValueError):
        crosscheck.check_fixtures(path)


@pytest.mark.gpu
def test_native_export_cross_checks_on_gpu(cuda):
    if not NATIVE.exists():
        pytest.fail(f"{NATIVE} is not built; run python tests/native/build.py")
    print("crosscheck: native driver --export-json", flush=True)
    result = subprocess.run([sys.executable, str(HERE / "native" / "crosscheck.py"), "--native-test", str(NATIVE)],
                            capture_output=True, text=True, timeout=110)
    print(result.stdout[-3000:], result.stderr[-3000:], flush=True)
    assert result.returncode == 0
    assert "GPU fixtures agree" in result.stdout
