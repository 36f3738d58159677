"""The native check program (tests/native/tilemix_native.cpp) and its JSON Lines
export, cross-checked by tests/native/fixture_check.py.

CPU: the program's validation table and closed forms (--cpu-only, no HIP
runtime call), its case list, the checker's self-validation, and the checker
accepting a correct record and rejecting a wrong, truncated or malformed one.
GPU: every dense and routed case through the reference's C++ API, exported and
recomputed independently on the CPU.
"""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "native"))
import fixture_check  # noqa: E402

NATIVE = HERE / "native" / "_build" / "tilemix_native"


def _native():
    if not NATIVE.exists():
        pytest.fail(f"{NATIVE} is not built; run python tests/native/build.py")
    return str(NATIVE)


def test_native_cpu_mode_makes_no_runtime_call():
    out = subprocess.run([_native(), "--cpu-only"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert "PASS API validation: 29 expectations, no HIP runtime call made" in out.stdout
    assert "PASS closed forms: 5 patterns against the fp64 oracle" in out.stdout


def test_native_case_list():
    out = subprocess.run([_native(), "--list"], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    cases = out.stdout.splitlines()
    assert len(cases) == 16 + 25 + 27
    assert sum("routes=none" in c for c in cases) == 41
    assert sum("routes=mixed" in c for c in cases) == 9
    assert any("stream=default" in c for c in cases)
    only = subprocess.run([_native(), "--list", "--only", "g=3"], capture_output=True, text=True, timeout=60)
    assert len(only.stdout.splitlines()) == 3


def test_checker_validates_itself():
    fixture_check.validate()


def _record(routed: bool):
    rng = np.random.default_rng(3)
    m, n, d = 20, 40, 8
    q, k, v = (rng.standard_normal((rows, d)).astype(np.float16) for rows in (m, n, n))
    scale = float(np.float32(1 / np.sqrt(d)))
    routes = rng.integers(0, 2, ((m + 15) // 16, (n + 31) // 32)).astype(np.uint8) if routed else None
    rec = fixture_check.Record(m, n, d, "random", q, k, v, np.zeros((m, d), np.float32), scale, routes)
    rec.o = fixture_check.expected(rec).astype(np.float32)
    obj = {"m": m, "n": n, "d": d, "pattern": "random", "q": q.astype(float).ravel().tolist(),
           "k": k.astype(float).ravel().tolist(), "v": v.astype(float).ravel().tolist(),
           "o": rec.o.astype(float).ravel().tolist(), "scale": scale}
    if routed:
        obj["routes"] = "".join(str(int(x)) for x in routes.ravel())
    return obj


@pytest.mark.parametrize("routed", [False, True])
def test_checker_accepts_and_rejects(tmp_path, routed):
    good = _record(routed)
    path = tmp_path / "good.jsonl"
    path.write_text(json.dumps(good) + "\n" + json.dumps(good) + "\n")
    assert fixture_check.check_file(path) == 2
    bad = dict(good, o=[x + 1e-3 for x in good["o"]])
    path = tmp_path / "bad.jsonl"
    path.write_text(json.dumps(bad) + "\n")
    with pytest.raises(AssertionError):
        fixture_check.check_file(path)
    for broken in ({k: v for k, v in good.items() if k != "o"}, dict(good, q=good["q"][:-1]),
                   dict(good, routes="2" * 6)):
        if "routes" in broken and not routed:
            continue
        path = tmp_path / "broken.jsonl"
        path.write_text(json.dumps(broken) + "\n")
        with pytest.raises(ValueError):
            fixture_check.check_file(path)


@pytest.mark.gpu
def test_native_program_and_export_on_gpu(cuda, tmp_path):
    path = tmp_path / "cases.jsonl"
    print("native program: every case, --export-json", flush=True)
    result = subprocess.run([_native(), "--export-json", str(path)], capture_output=True, text=True, timeout=110)
    print(result.stdout[-3000:], result.stderr[-3000:], flush=True)
    assert result.returncode == 0
    assert "PASS GPU cases: 41 dense + 27 routed" in result.stdout
    assert fixture_check.check_file(path) == 68
