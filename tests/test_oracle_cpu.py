"""Pins the C oracle (oracle/tilemix_oracle.c) on the CPU.

The oracle is the checker of every GPU parity test, so each of its functions
is checked here against something that does not share its code:

* fp16 conversions: numpy's binary16 (exhaustive for half -> float, the
  rounding cases and a large random sample for float -> half);
* mt19937: the C++ standard's known answer (10000th output of seed 5489 is
  4123659995, [rand.predef]), a fixture written by libstdc++'s std::mt19937
  (tests/golden/make_golden.py) and numpy's MT19937 with the same seeding;
* the input patterns of src/tests/tilemix_test.cu:43-134, restated in numpy;
* the quantizer: the known tie answers of src/tests/tilemix_test.cu:376-386,
  closed forms of the zeros / tiny / max-range cases (:366-381), invariants
  that any correct symmetric quantizer meets, and a numpy float32 brute force;
* int8 dots: numpy integer matmul and the max-int8 closed form (+-127^2 d);
* dense attention: the closed forms of src/tests/tilemix_test.cu:237-260 and
  :343-353, and a numpy float64 softmax;
* the mixed TileMix path and its skip / causal extensions: numpy float64
  brute force and the definitional equivalences (all-FP16 routes == dense,
  skip == keys removed, causal == masked dense).

A planted mistake (wrong rounding, a dropped scale, a transposed operand, an
off-by-one in a mask) fails at least one of these.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build()


def as_f16_bits(values) -> np.ndarray:
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def from_bits(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float64)


# ------------------------------------------------------------------- fp16


def test_half_to_float_exhaustive():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = oracle.half_to_float(bits)
    theirs = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(theirs)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), theirs[~nan].view(np.uint32))


def test_float_to_half_rounding():
    rng = np.random.default_rng(1)
    raw = rng.integers(0, 1 << 32, size=1 << 21, dtype=np.uint64).astype(np.uint32).view(np.float32)
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e9, np.inf, -np.inf,
                        2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26, 2.0 ** -14,
                        2.0 ** -14 - 2.0 ** -25, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11,
                        0.1, -0.1, 1.0 / 3.0], dtype=np.float32)
    with np.errstate(all="ignore"):
        values = np.concatenate([raw, special, raw / np.float32(2.0 ** 100)])
    values = values[~np.isnan(values)]
    ours = oracle.float_to_half(values)
    with np.errstate(all="ignore"):
        theirs = values.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, theirs)
    nan = oracle.float_to_half(np.array([np.nan], dtype=np.float32))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x03FF) != 0


# --------------------------------------------------------------- mt19937


def test_mt19937_standard_known_answer():
    # [rand.predef]: the 10000th consecutive output of a default-constructed mt19937.
    assert int(oracle.mt19937_outputs(5489, 10000)[-1]) == 4123659995


def test_mt19937_matches_libstdcxx_fixture():
    fixture = json.loads((GOLDEN / "mt19937_libstdcxx.json").read_text())
    assert len(fixture["entries"]) >= 5
    for entry in fixture["entries"]:
        ours = oracle.mt19937_outputs(entry["seed"], 10000)
        assert ours[: len(entry["first"])].tolist() == entry["first"], entry["seed"]
        assert int(ours[-1]) == entry["output_10000"], entry["seed"]


@pytest.mark.parametrize("seed", [0, 1, 5489, 2236, 17 * 131 + 65 * 17 + 1, 0xFFFFFFFF])
def test_mt19937_matches_numpy(seed):
    raw = np.random.RandomState(seed)._bit_generator.random_raw(3000)
    assert np.array_equal(oracle.mt19937_outputs(seed, 3000), raw.astype(np.uint32))


# ---------------------------------------------------------- input patterns


def numpy_inputs(m: int, n: int, d: int, pattern: str):
    """Restatement of src/tests/tilemix_test.cu:43-134 with numpy's MT19937."""
    gen = np.random.RandomState(m * 131 + n * 17 + d)._bit_generator
    raw = gen.random_raw(m * d + 2 * n * d).astype(np.int64)
    values = ((raw % 20001) - 10000).astype(np.float32) / np.float32(10000.0)
    q = values[: m * d].reshape(m, d).copy()
    k = values[m * d: m * d + n * d].reshape(n, d).copy()
    v = values[m * d + n * d:].reshape(n, d).copy()
    if pattern == "random":
        pass
    elif pattern == "zeros":
        q[:], k[:], v[:] = 0, 0, 0
    elif pattern == "block-outliers":
        q[127, 0], q[128, 0], k[63, 0], k[128, 0] = 8.0, 0.125, -16.0, 0.25
    elif pattern == "max-int8":
        q[:], k[:] = 1.0, 1.0
        k[0, :] = -1.0
    elif pattern == "zero-v":
        v[:] = 0
    elif pattern == "constant-v":
        v[:] = ((np.arange(d) % 7 - 3) * 0.25)[None, :]
    elif pattern == "cancellation":
        q[:] = 0
        v[:] = np.where(np.arange(n) % 2 == 1, -1.0, 1.0)[:, None]
    elif pattern == "large-dot":
        q[:] = 1000.0
        k[:] = -1000.0
        k[0, :] = 1000.0
    else:
        q[:] = 0
        if pattern != "uniform":
            k[:] = 0
            q[:, 0] = 1.0
            tile = np.arange(n) // 32
            if pattern == "rising":
                score, value = 4.0 * (tile - 1), np.where(tile == 0, 1.0, np.where(tile == 1, -1.0, 2.0))
            elif pattern == "falling":
                score, value = 4.0 * (1 - tile), np.where(tile == 0, 1.0, np.where(tile == 1, -1.0, 2.0))
            elif pattern == "alternating":
                score = np.array([0, 4, -2, 8, 10], dtype=np.float64)[tile]
                value = np.array([1, -1, 2, -2, 3], dtype=np.float64)[tile]
            elif pattern == "late-extreme":
                last = np.arange(n) == n - 1
                score, value = np.where(last, 1000.0, 0.0), np.where(last, 3.0, 1.0)
            elif pattern == "negative":
                score, value = np.full(n, -1000.0), (np.arange(n) % 7 - 3) * 0.25
            else:
                raise ValueError(pattern)
            k[:, 0] = score
            v[:] = np.asarray(value, dtype=np.float32)[:, None]
    return as_f16_bits(q), as_f16_bits(k), as_f16_bits(v)


PATTERN_SHAPES = [
    (33, 47, 8, "random"), (137, 73, 31, "random"), (64, 64, 64, "zeros"), (129, 131, 17, "block-outliers"),
    (17, 65, 9, "max-int8"), (40, 70, 16, "zero-v"), (40, 70, 16, "constant-v"), (40, 70, 16, "cancellation"),
    (20, 33, 4, "large-dot"), (20, 33, 4, "uniform"), (17, 65, 1, "rising"), (17, 65, 1, "falling"),
    (17, 129, 1, "alternating"), (17, 65, 1, "late-extreme"), (17, 65, 1, "negative"),
]


@pytest.mark.parametrize("m,n,d,pattern", PATTERN_SHAPES)
def test_make_inputs_matches_numpy_restatement(m, n, d, pattern):
    ours = oracle.make_inputs(m, n, d, pattern)
    theirs = numpy_inputs(m, n, d, pattern)
    for name, a, b in zip("qkv", ours, theirs):
        assert np.array_equal(a, b), f"{pattern} {name}"


def test_make_inputs_rejects_unknown_and_small_outlier_shapes():
    with pytest.raises(ValueError):
        oracle.make_inputs(4, 4, 4, "no-such-pattern")
    with pytest.raises(ValueError):
        oracle.make_inputs(64, 64, 4, "block-outliers")   # needs two quantization blocks
    with pytest.raises(ValueError):
        oracle.make_inputs(17, 193, 1, "alternating")     # five 32-key tiles at most


# -------------------------------------------------------------- quantizer


def numpy_quantize(bits: np.ndarray, block_rows: int):
    """Symmetric block quantizer in numpy float32 (IEEE single, round to nearest)."""
    x = bits.view(np.float16).astype(np.float32)
    rows = x.shape[0]
    out = np.zeros(x.shape, dtype=np.int8)
    scales = []
    for first in range(0, rows, block_rows):
        block = x[first:first + block_rows]
        scale = np.float32(np.abs(block).max()) / np.float32(127.0)
        scales.append(np.float16(scale).view(np.uint16))
        if scale == 0:
            continue
        ratio = block / scale
        shifted = np.where(ratio < 0, ratio - np.float32(0.5), ratio + np.float32(0.5)).astype(np.float32)
        out[first:first + block_rows] = np.clip(np.trunc(shifted), -127, 127).astype(np.int8)
    return out, np.array(scales, dtype=np.uint16)


def test_quantizer_known_ties():
    # src/tests/tilemix_test.cu:373-386: values at the rounding ties and their known bytes.
    ties = np.array([127, -127, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5], dtype=np.float32)
    x = as_f16_bits(np.resize(ties, 129).reshape(129, 1))
    values, scales = oracle.quantize(x, 128)
    assert values[:8, 0].tolist() == [127, -127, 1, -1, 2, -2, 127, -127]
    assert scales.tolist() == [0x3C00, 0x3C00]  # amax 127 -> scale exactly 1.0 in both blocks
    assert values[128, 0] == 127


def test_quantizer_zero_block():
    x = np.zeros((129, 17), dtype=np.uint16)
    for block in (128, 64):
        values, scales = oracle.quantize(x, block)
        assert not values.any() and not scales.any()
    # A zero block next to a non-zero one keeps its zero scale and bytes.
    x[70:, :] = as_f16_bits(np.full((59, 17), 0.75))
    values, scales = oracle.quantize(x, 64)
    assert scales[0] == 0 and not values[:64].any()
    assert (values[70:] == 127).all()


def test_quantizer_tiny_and_max_range():
    # src/tests/tilemix_test.cu:378-381. Tiny: +-2^-24 gives a scale that
    # underflows to fp16 zero, yet the bytes are +-127 (quantized with the fp32
    # scale). Max range: +-65504 gives +-127 and scale RN16(65504/127) = 516.
    signs = np.where(np.arange(129 * 3) % 2 == 1, -1.0, 1.0).reshape(129, 3)
    tiny = as_f16_bits(signs * 2.0 ** -24)
    values, scales = oracle.quantize(tiny, 128)
    assert np.array_equal(values, (signs * 127).astype(np.int8))
    assert scales.tolist() == [0, 0]
    signs = np.where(np.arange(5 * 128) % 2 == 1, -1.0, 1.0).reshape(5, 128)
    big = as_f16_bits(signs * 65504.0)
    values, scales = oracle.quantize(big, 64)
    assert np.array_equal(values, (signs * 127).astype(np.int8))
    assert from_bits(scales).tolist() == [516.0]


def test_quantizer_special_values():
    # src/tilemix.cu:27,45: the block maximum skips NaNs (fmaxf), and the
    # saturating __float2int_rz turns a NaN quotient into 0, so NaN elements,
    # and +-inf elements of a block whose maximum is inf (inf / inf), give 0.
    nan, neg_nan, inf, neg_inf = 0x7E00, 0xFE00, 0x7C00, 0xFC00
    x = as_f16_bits(np.full((320, 8), 0.5))
    x[3, 2], x[7, 1] = nan, neg_nan          # block 0: NaNs among 0.5s
    x[64 + 5, 4] = inf                       # block 1: an inf maximum
    x[128:192] = nan                         # block 2: NaN only
    x[192 + 1, 0], x[192 + 9, 6] = nan, neg_inf  # block 3: NaN and -inf
    x[256:320] = 0x8000                      # block 4: -0 only
    values, scales = oracle.quantize(x, 64)
    assert scales.tolist() == [int(as_f16_bits(np.float32(0.5) / np.float32(127.0))), inf, 0, inf, 0]
    expected = np.zeros((320, 8), dtype=np.int8)
    expected[:64] = 127
    expected[3, 2] = expected[7, 1] = 0
    assert np.array_equal(values, expected)


@pytest.mark.parametrize("rows,d,block", [(137, 31, 128), (73, 31, 64), (300, 128, 128), (257, 64, 64),
                                          (131, 17, 64), (5, 1, 64)])
def test_quantizer_brute_force_and_invariants(rows, d, block):
    rng = np.random.default_rng(rows * d)
    x = rng.standard_t(3, size=(rows, d)).astype(np.float32)
    x[rng.random((rows, d)) < 0.05] *= 40.0
    bits = as_f16_bits(x)
    values, scales = oracle.quantize(bits, block)
    ref_values, ref_scales = numpy_quantize(bits, block)
    assert np.array_equal(values, ref_values) and np.array_equal(scales, ref_scales)
    xf = from_bits(bits)
    for b, first in enumerate(range(0, rows, block)):
        blk, q = xf[first:first + block], values[first:first + block].astype(np.float64)
        amax = np.abs(blk).max()
        s = float(np.float32(amax) / np.float32(127.0))
        assert abs(from_bits(scales[b:b + 1])[0] - s) <= 2.0 ** -11 * s + 2.0 ** -24
        assert np.abs(q).max() == 127
        # round half away from zero of x/s, up to fp32 rounding of the ratio
        assert np.all(np.abs(q - blk / s) <= 0.5 + 1e-5)
        assert np.all(np.sign(q) * np.sign(blk) >= 0)


def test_quantizer_block_outliers():
    # src/tests/tilemix_test.cu:63-70: an outlier decides its own block's scale only.
    q, k, _ = oracle.make_inputs(129, 131, 17, "block-outliers")
    q8, qs = oracle.quantize(q, 128)
    k8, ks = oracle.quantize(k, 64)
    assert from_bits(qs).tolist()[0] == float(np.float16(np.float32(8.0) / np.float32(127)))
    assert from_bits(ks).tolist()[0] == float(np.float16(np.float32(16.0) / np.float32(127)))
    assert q8[127, 0] == 127 and k8[63, 0] == -127
    row128 = np.float32(np.abs(from_bits(q[128])).max())
    assert from_bits(qs)[1] == float(np.float16(row128 / np.float32(127))) < from_bits(qs)[0]


# ------------------------------------------------------------------- dots


def test_int8_dot_matches_numpy():
    rng = np.random.default_rng(3)
    for d in (1, 17, 64, 128):
        q8 = rng.integers(-127, 128, size=(9, d), dtype=np.int8)
        k8 = rng.integers(-127, 128, size=(11, d), dtype=np.int8)
        ref = q8.astype(np.int64) @ k8.astype(np.int64).T
        for i in range(9):
            for j in range(11):
                assert oracle.int8_dot(q8, k8, i, j) == ref[i, j]


def test_int8_dot_max_closed_form():
    # src/tests/tilemix_test.cu:71-76: all-ones Q and K with K row 0 negated
    # quantize to +-127, so the dots are +-127^2 d (|dot| <= 2,064,512 at d=128).
    q, k, _ = oracle.make_inputs(17, 65, 128, "max-int8")
    q8, _ = oracle.quantize(q, 128)
    k8, _ = oracle.quantize(k, 64)
    assert oracle.int8_dot(q8, k8, 3, 0) == -127 * 127 * 128 == -2064512
    assert oracle.int8_dot(q8, k8, 16, 64) == 127 * 127 * 128


# ------------------------------------------------------- dense attention


def numpy_attention(q, k, v, scale=None, mask=None):
    """float64 softmax(scale Q K^T) V over fp16 bit inputs; mask True = visible.
    Without ``scale`` it is the dense reference's double 1/sqrt(d)."""
    qf, kf, vf = from_bits(q), from_bits(k), from_bits(v)
    scale = 1.0 / math.sqrt(qf.shape[1]) if scale is None else float(np.float32(scale))
    s = (qf @ kf.T) * scale
    if mask is not None:
        s = np.where(mask, s, -np.inf)
    out = np.zeros((qf.shape[0], vf.shape[1]))
    for i in range(qf.shape[0]):
        if not np.isfinite(s[i]).any():
            continue
        p = np.exp(s[i] - s[i].max())
        out[i] = (p / p.sum()) @ vf
    return out


def test_dense_closed_forms():
    # src/tests/tilemix_test.cu:237-260 (rows of 17 queries, d = 1).
    e = math.exp
    expected = {
        "rising": (32 * e(-8) - 32 * e(-4) + 2) / (32 * e(-8) + 32 * e(-4) + 1),
        "falling": (32 - 32 * e(-4) + 2 * e(-8)) / (32 + 32 * e(-4) + e(-8)),
        "alternating": (32 * e(-10) - 32 * e(-6) + 2 * 32 * e(-12) - 2 * 32 * e(-2) + 3)
        / (32 * e(-10) + 32 * e(-6) + 32 * e(-12) + 32 * e(-2) + 1),
        "late-extreme": 3.0,
    }
    for pattern, value in expected.items():
        n = 129 if pattern == "alternating" else 65
        q, k, v = oracle.make_inputs(17, n, 1, pattern)
        out = oracle.attention(q, k, v)
        assert np.allclose(out, value, rtol=1e-12, atol=1e-12), pattern
    q, k, v = oracle.make_inputs(17, 65, 1, "negative")
    assert np.allclose(oracle.attention(q, k, v), from_bits(v).mean(), rtol=1e-12, atol=1e-12)


def test_dense_special_cases():
    # Zero Q -> mean of V; one key -> that V row; q = 1000, k = +-1000 picks the
    # single aligned key (python/reference_attention.py:44-52 checks the same).
    q, k, v = oracle.make_inputs(5, 9, 8, "cancellation")
    assert np.allclose(oracle.attention(q, k, v), from_bits(v).mean(axis=0), atol=1e-15)
    rng = np.random.default_rng(4)
    q1 = as_f16_bits(rng.standard_normal((6, 16)))
    k1 = as_f16_bits(rng.standard_normal((1, 16)))
    v1 = as_f16_bits(rng.standard_normal((1, 16)))
    assert np.array_equal(oracle.attention(q1, k1, v1), np.repeat(from_bits(v1), 6, axis=0))
    q, k, v = oracle.make_inputs(3, 5, 4, "large-dot")
    assert np.allclose(oracle.attention(q, k, v), from_bits(v)[0][None, :], atol=0)


@pytest.mark.parametrize("m,n,d", [(33, 47, 8), (64, 129, 64), (17, 300, 128)])
def test_dense_matches_numpy(m, n, d):
    q, k, v = oracle.make_inputs(m, n, d, "random")
    assert np.allclose(oracle.attention(q, k, v), numpy_attention(q, k, v), rtol=1e-12, atol=1e-13)


def test_dense_rejects_non_finite():
    q, k, v = oracle.make_inputs(4, 4, 4, "random")
    k = k.copy()
    k[1, 2] = 0x7C00
    with pytest.raises(ValueError):
        oracle.attention(q, k, v)


def test_score_scale_closed_form():
    # src/tests/tilemix_test.cu:330-353: q = 1, k = (-1, 0, 1), v = (2, 4, 8).
    q = as_f16_bits([[1.0]])
    k = as_f16_bits([[-1.0], [0.0], [1.0]])
    v = as_f16_bits([[2.0], [4.0], [8.0]])
    for scale in (1.0, 0.0, -1.0, 0.5):
        a, b = math.exp(-scale), math.exp(scale)
        expected = (2 * a + 4 + 8 * b) / (a + 1 + b)
        out = oracle.tilemix(q, k, v, score_scale=scale)
        assert abs(out[0, 0] - expected) <= 1e-14, scale


# ------------------------------------------------------------- tilemix


def random_problem(m, n, d, seed):
    q, k, v = oracle.make_inputs(m, n, d, "random")
    rng = np.random.default_rng(seed)
    routes = rng.integers(0, 2, size=((m + 15) // 16, (n + 31) // 32), dtype=np.uint8)
    q8, qs = oracle.quantize(q, 128)
    k8, ks = oracle.quantize(k, 64)
    return q, k, v, q8, k8, qs, ks, routes


def numpy_tilemix(q, k, v, q8, k8, qs, ks, routes, scale, causal=False):
    """reference_tilemix.h:53-90 in numpy float64: INT8 cells score the exact
    integer dot times both fp16 block scales; skip cells and (if causal) keys
    after the query are removed."""
    m, n = q.shape[0], k.shape[0]
    cell = np.repeat(np.repeat(routes, 16, axis=0)[:m], 32, axis=1)[:, :n]
    dots = q8.astype(np.int64) @ k8.astype(np.int64).T
    qscale = from_bits(qs)[np.arange(m) // 128][:, None]
    kscale = from_bits(ks)[np.arange(n) // 64][None, :]
    fp = from_bits(q) @ from_bits(k).T
    # score_scale crosses the reference API as a C float (reference_tilemix.h:72)
    s = np.where(cell == 1, dots * qscale * kscale, fp) * float(np.float32(scale))
    visible = cell != 2
    if causal:
        visible &= np.arange(n)[None, :] <= np.arange(m)[:, None]
    s = np.where(visible, s, -np.inf)
    out = np.zeros((m, q.shape[1]))
    vf = from_bits(v)
    for i in range(m):
        if visible[i].any():
            p = np.exp(s[i] - s[i].max())
            out[i] = (p / p.sum()) @ vf
    return out


@pytest.mark.parametrize("m,n,d", [(17, 65, 1), (129, 131, 17), (200, 70, 64), (64, 257, 128)])
def test_tilemix_matches_numpy(m, n, d):
    q, k, v, q8, k8, qs, ks, routes = random_problem(m, n, d, seed=m + n)
    scale = 1.0 / math.sqrt(d)
    out = oracle.tilemix(q, k, v, q8, k8, qs, ks, routes, scale)
    assert np.allclose(out, numpy_tilemix(q, k, v, q8, k8, qs, ks, routes, scale), rtol=1e-12, atol=1e-13)


def test_tilemix_all_fp16_equals_dense():
    # src/tests/tilemix_test.cu:506-509: all-FP16 routing is the dense path.
    q, k, v, q8, k8, qs, ks, routes = random_problem(70, 90, 32, seed=1)
    zero = np.zeros_like(routes)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(32)))
    routed = oracle.tilemix(q, k, v, q8, k8, qs, ks, zero, scale)
    assert np.array_equal(routed, oracle.tilemix(q, k, v, score_scale=scale))
    assert np.allclose(routed, oracle.attention(q, k, v), rtol=1e-6, atol=1e-7)  # fp32 vs fp64 1/sqrt(d)


def test_tilemix_int8_uses_both_scales():
    # Doubling one K block's fp16 scale must change exactly the scores of that
    # block's keys: a dropped or swapped scale term fails this.
    q, k, v, q8, k8, qs, ks, routes = random_problem(40, 130, 16, seed=2)
    ones = np.ones_like(routes)
    base = oracle.tilemix(q, k, v, q8, k8, qs, ks, ones, 0.25)
    ks2 = ks.copy()
    ks2[1] = as_f16_bits([from_bits(ks[1:2])[0] * 2])[0]
    changed = oracle.tilemix(q, k, v, q8, k8, qs, ks2, ones, 0.25)
    assert np.allclose(changed, numpy_tilemix(q, k, v, q8, k8, qs, ks2, ones, 0.25), rtol=1e-12, atol=1e-13)
    assert not np.allclose(base, changed)


def test_tilemix_skip_equals_removed_keys():
    q, k, v, q8, k8, qs, ks, routes = random_problem(48, 128, 16, seed=3)
    routes[:, 1] = 2  # keys 32..63 skipped for every query
    out = oracle.tilemix(q, k, v, q8, k8, qs, ks, routes, 0.3)
    keep = np.r_[0:32, 64:128]
    kept_routes = np.delete(routes, 1, axis=1)
    # Without keys 32..63 the key blocks shift, so compare through numpy on the kept keys.
    expected = numpy_tilemix(q, k, v, q8, k8, qs, ks, routes, 0.3)
    assert np.allclose(out, expected, rtol=1e-12, atol=1e-13)
    fp16_rows = oracle.tilemix(q, k[keep], v[keep], score_scale=0.3,
                               routes=np.zeros_like(kept_routes))
    fp16_out = oracle.tilemix(q, k, v, q8, k8, qs, ks, np.where(routes == 2, 2, 0).astype(np.uint8), 0.3)
    assert np.allclose(fp16_out, fp16_rows, rtol=1e-12, atol=1e-13)


def test_tilemix_all_skipped_row_is_zero():
    q, k, v, q8, k8, qs, ks, routes = random_problem(32, 64, 8, seed=4)
    routes[0, :] = 2
    out = oracle.tilemix(q, k, v, q8, k8, qs, ks, routes, 0.5)
    assert not out[:16].any() and out[16:].any()


def test_tilemix_causal_equals_masked_dense():
    q, k, v = oracle.make_inputs(77, 77, 24, "random")
    scale = 1.0 / math.sqrt(24)
    out = oracle.tilemix(q, k, v, score_scale=scale, causal=True)
    mask = np.arange(77)[None, :] <= np.arange(77)[:, None]
    assert np.allclose(out, numpy_attention(q, k, v, scale, mask), rtol=1e-12, atol=1e-13)
    # Row 0 sees key 0 only.
    assert np.array_equal(out[0], from_bits(v)[0])


def test_tilemix_row_subset():
    q, k, v, q8, k8, qs, ks, routes = random_problem(150, 100, 16, seed=5)
    full = oracle.tilemix(q, k, v, q8, k8, qs, ks, routes, 0.25, causal=True)
    rows = np.array([149, 0, 77, 128, 3], dtype=np.int32)
    part = oracle.tilemix(q, k, v, q8, k8, qs, ks, routes, 0.25, causal=True, rows=rows)
    assert np.array_equal(part, full[rows])


# ----------------------------------------------------------- route decode


def test_decode_routes_matches_independent_packer():
    from helpers import reference_group_words

    for m, n, g, pattern in [(17, 2049, 1, "mixed"), (40, 4097, 2, "mixed"), (33, 700, 3, "int8-requested"),
                             (16, 32, 1, "fp16"), (100, 9000, 5, "mixed")]:
        qt, kt = (m + 15) // 16, (n + 31) // 32
        words, bits = reference_group_words(qt, kt, g, pattern)
        decoded = oracle.decode_routes(words, None, m, n, g)
        assert np.array_equal(decoded, bits), (m, n, g, pattern)
        skip_words, skip_bits = reference_group_words(qt, kt, g, "mixed")
        both = oracle.decode_routes(words, skip_words, m, n, g)
        assert np.array_equal(both, np.where(skip_bits == 1, 2, bits)), (m, n, g, pattern)
