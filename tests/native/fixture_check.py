"""Independent cross-check of the native driver's JSON Lines export (test code).

The native program (tests/native/tilemix_native.cpp) runs every GPU case through
the reference's C++ API and, with ``--export-json FILE``, writes one JSON
object per case: ``m``, ``n``, ``d``, ``pattern``, ``q``, ``k``, ``v`` (fp16
values), ``o`` (the fp32 GPU output) and ``scale``, plus ``routes`` (one
character per 16 x 32 cell, '1' = INT8) for a routed case. This module
recomputes each record's output on the CPU with code that shares nothing with
the native program's checker:

* a record without ``routes``: softmax(scale Q K^T) V in numpy float64;
* a routed record: the TileMix mixed path, with INT8 cells scored from the
  quantized operands - the quantizer and the exact int32 dots restated here in
  numpy (fp32 abs-max / 127, the fp16-rounded scale for dequantisation,
  round-half-away), the scores and softmax in float64 (the fp64 TileMix
  definition of src/tests/reference_tilemix.h:53-90);

and requires |o - expected| <= 1e-5 + 1e-4 |expected| for every element (the
reference's rule, src/tests/tilemix_test.cu:137-155).

``validate()`` pins this module's own arithmetic first: the dense path against
three closed forms (zero queries give the mean of V, one key gives its V row,
well-separated logits give the winning V row) and against the C oracle
(oracle.attention) on seeded shapes; the routed path with every cell FP16
against the dense path, and with INT8 cells against oracle.tilemix.

Usage: python tests/native/fixture_check.py FILE.jsonl
       python tests/native/fixture_check.py --run tests/native/_build/tilemix_native
"""
from __future__ import annotations

import argparse
import json
import subprocess
import sys
import tempfile
from dataclasses import dataclass
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
REQUIRED = ("m", "n", "d", "pattern", "q", "k", "v", "o")
ATOL, RTOL = 1e-5, 1e-4


@dataclass
class Record:
    m: int
    n: int
    d: int
    pattern: str
    q: np.ndarray  # float16 [m, d]
    k: np.ndarray  # float16 [n, d]
    v: np.ndarray  # float16 [n, d]
    o: np.ndarray  # float32 [m, d]
    scale: float
    routes: np.ndarray | None  # uint8 [ceil(m/16), ceil(n/32)], 1 = INT8

    @property
    def label(self) -> str:
        kind = "routed" if self.routes is not None else "dense"
        return f"M={self.m} N={self.n} d={self.d} pattern={self.pattern} {kind}"


def parse(line: str, where: str = "") -> Record:
    obj = json.loads(line)
    missing = [key for key in REQUIRED if key not in obj]
    if missing:
        raise ValueError(f"{where}: record lacks {missing}")
    m, n, d = int(obj["m"]), int(obj["n"]), int(obj["d"])

    def matrix(key, rows, dtype):
        values = np.asarray(obj[key], dtype=np.float64)
        if values.size != rows * d:
            raise ValueError(f"{where}: '{key}' holds {values.size} values, expected {rows * d}")
        return values.astype(dtype).reshape(rows, d)

    routes = None
    if "routes" in obj:
        rows, cols = (m + 15) // 16, (n + 31) // 32
        text = obj["routes"]
        if len(text) != rows * cols or set(text) - {"0", "1"}:
            raise ValueError(f"{where}: 'routes' must be {rows * cols} characters of 0/1")
        routes = (np.frombuffer(text.encode(), dtype=np.uint8) - ord("0")).reshape(rows, cols)
    return Record(m, n, d, str(obj["pattern"]), matrix("q", m, np.float16), matrix("k", n, np.float16),
                  matrix("v", n, np.float16), matrix("o", m, np.float32),
                  float(obj.get("scale", 1.0 / np.sqrt(d))), routes)


def softmax_rows(scores: np.ndarray) -> np.ndarray:
    shifted = scores - scores.max(axis=1, keepdims=True)
    weights = np.exp(shifted)
    return weights / weights.sum(axis=1, keepdims=True)


def dense(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """softmax(scale Q K^T) V, all in float64."""
    scores = (q.astype(np.float64) @ k.astype(np.float64).T) * scale
    return softmax_rows(scores) @ v.astype(np.float64)


def quantize_blocks(x: np.ndarray, block_rows: int) -> tuple[np.ndarray, np.ndarray]:
    """Per block of rows: scale = fp32(absmax / 127), bytes = clamp(trunc(x / scale +- 0.5), +-127)
    computed in fp32; returns the bytes and the fp16-rounded scales used to dequantise."""
    x32 = x.astype(np.float32)
    out = np.zeros(x.shape, dtype=np.int8)
    scales = np.zeros((x.shape[0] + block_rows - 1) // block_rows, dtype=np.float16)
    for b in range(scales.size):
        block = x32[b * block_rows:(b + 1) * block_rows]
        finite = np.abs(block)[~np.isnan(block)]
        scale = np.float32(finite.max() if finite.size else 0.0) / np.float32(127.0)
        scales[b] = np.float16(scale)
        if scale > 0:
            with np.errstate(invalid="ignore"):
                ratio = block / np.float32(scale)
                rounded = np.trunc(ratio + np.copysign(np.float32(0.5), ratio))
            out[b * block_rows:(b + 1) * block_rows] = np.nan_to_num(np.clip(rounded, -127, 127)).astype(np.int8)
    return out, scales


def tilemix(rec: Record) -> np.ndarray:
    """The routed (mixed INT8/FP16) path in float64 over exact integer dots."""
    q8, q_scales = quantize_blocks(rec.q, 128)
    k8, k_scales = quantize_blocks(rec.k, 64)
    dots = q8.astype(np.int64) @ k8.astype(np.int64).T
    rows = np.arange(rec.m)
    cols = np.arange(rec.n)
    int8_cell = rec.routes[rows[:, None] // 16, cols[None, :] // 32].astype(bool)
    # ((dot * q_scale) * k_scale) * scale in float64, the fp64 TileMix definition
    # (src/tests/reference_tilemix.h:53-90).
    qs = q_scales.astype(np.float64)[rows // 128][:, None]
    ks = k_scales.astype(np.float64)[cols // 64][None, :]
    int8_scores = ((dots.astype(np.float64) * qs) * ks) * rec.scale
    fp16_scores = (rec.q.astype(np.float64) @ rec.k.astype(np.float64).T) * rec.scale
    scores = np.where(int8_cell, int8_scores, fp16_scores)
    return softmax_rows(scores) @ rec.v.astype(np.float64)


def expected(rec: Record) -> np.ndarray:
    return tilemix(rec) if rec.routes is not None else dense(rec.q, rec.k, rec.v, rec.scale)


def check(rec: Record) -> float:
    """Max abs error of the record's GPU output; raises AssertionError outside the rule."""
    want = expected(rec)
    got = rec.o.astype(np.float64)
    err = np.abs(got - want)
    bad = ~(np.isfinite(got) & (err <= ATOL + RTOL * np.abs(want)))
    if bad.any():
        i, j = np.argwhere(bad)[0]
        raise AssertionError(f"{rec.label}: o[{i},{j}] = {got[i, j]!r}, expected {want[i, j]!r}")
    return float(err.max())


def check_file(path: Path) -> int:
    count = 0
    with Path(path).open() as source:
        for number, line in enumerate(source, 1):
            if not line.strip():
                continue
            rec = parse(line, f"{path}:{number}")
            worst = check(rec)
            print(f"PASS {rec.label} max_abs_error={worst:.3g}")
            count += 1
    return count


def validate(seed: int = 20261202) -> None:
    """Pin this module's arithmetic before trusting it as a checker."""
    sys.path.insert(0, str(ROOT))
    import oracle

    h = lambda a: np.asarray(a, dtype=np.float16)
    v = h(np.arange(35).reshape(5, 7))
    assert np.allclose(dense(h(np.zeros((3, 7))), h(np.ones((5, 7))), v, 0.5), v.astype(np.float64).mean(0))
    assert np.allclose(dense(h(np.ones((2, 7))), h(np.ones((1, 7))), v[:1], 1.0), v[:1].astype(np.float64))
    assert np.allclose(dense(h([[1000.0]]), h([[1000.0], [-1000.0]]), h([[3.0], [-7.0]]), 1.0), [[3.0]])
    rng = np.random.default_rng(seed)
    for m, n, d in ((1, 1, 1), (3, 5, 7), (17, 33, 17), (40, 70, 64)):
        q, k, vv = (h(rng.standard_normal((rows, d))) for rows in (m, n, n))
        bits = lambda a: a.view(np.uint16)
        theirs = oracle.attention(bits(q), bits(k), bits(vv))
        assert np.allclose(dense(q, k, vv, 1.0 / np.sqrt(d)), theirs, atol=1e-12, rtol=1e-12), (m, n, d)
        cells = ((m + 15) // 16, (n + 31) // 32)
        scale = float(np.float32(1.0 / np.sqrt(d)))  # the library takes the scale as a float
        fp16 = Record(m, n, d, "seeded", q, k, vv, np.zeros((m, d), np.float32), scale, np.zeros(cells, np.uint8))
        assert np.array_equal(tilemix(fp16), dense(q, k, vv, fp16.scale))
        mixed = Record(**{**fp16.__dict__, "routes": rng.integers(0, 2, cells).astype(np.uint8)})
        q8, qs = oracle.quantize(bits(q), 128)
        k8, ks = oracle.quantize(bits(k), 64)
        assert np.array_equal(quantize_blocks(q, 128)[0], q8) and np.array_equal(quantize_blocks(k, 64)[0], k8)
        assert np.array_equal(quantize_blocks(q, 128)[1].view(np.uint16), qs)
        theirs = oracle.tilemix(bits(q), bits(k), bits(vv), q8, k8, qs, ks, mixed.routes, mixed.scale)
        assert np.allclose(tilemix(mixed), theirs, atol=1e-12, rtol=1e-9), (m, n, d)
    print("PASS fixture checker: closed forms, C oracle agreement (dense and routed)")


def run_native(executable: Path) -> int:
    """Run the native program with --export-json, then check every record it wrote."""
    with tempfile.TemporaryDirectory(prefix="tilemix-fixtures-") as directory:
        path = Path(directory) / "cases.jsonl"
        subprocess.run([str(Path(executable).resolve()), "--export-json", str(path)], check=True)
        count = check_file(path)
    if count == 0:
        raise RuntimeError("the native program exported no records")
    print(f"PASS {count} GPU records agree with the CPU recomputation")
    return count


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("jsonl", nargs="?", type=Path)
    parser.add_argument("--run", type=Path, help="native program to run with --export-json first")
    args = parser.parse_args()
    validate()
    if args.run:
        run_native(args.run)
    if args.jsonl:
        print(f"PASS {check_file(args.jsonl)} records of {args.jsonl}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
