"""GPU parity suite restating the reference's native test binary
(src/tests/tilemix_test.cu:263-614) through the C ABI:

* 41 dense cases vs the fp64 oracle at 1e-5 + 1e-4|x| with output guards,
  input immutability and default / non-default streams (:263-328, :592-605);
* 4 analytic score-scale cases with buffer reuse (:330-355);
* 6 quantizer cases, bytes/scales/guards bit-exact (:364-422);
* 80 routing cases: exact int32 dots, decoded trace bits, all-FP16 == un-routed
  bitwise, mixed output vs the fp64 TileMix oracle (:424-578).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from helpers import (GUARD_DOT, GUARD_F32, GUARD_I8, GUARD_SCALE, GUARD_TRACE, compare, dev, dev_half,
                     guarded, guarded_lead, host, nan_padded_rows, reference_group_words)

pytestmark = pytest.mark.gpu

INT_MAX = 2**31 - 1

# The head-dimension sweep covers each kernel layout class: padded and rotated
# K / V rows, 64- and 128-byte K8 rows, and (d % 16 == 0, aligned runs) the
# vector path of every padded head dimension 32 * ceil(d / 32).
DENSE_CASES = [(3, 33, d, "random", False)
               for d in (1, 15, 16, 17, 31, 32, 33, 48, 49, 63, 64, 65, 80, 81, 96, 97, 112, 113, 127, 128)] + [
    (1, 1, 1, "random", False), (3, 5, 7, "random", False), (15, 31, 15, "random", False),
    (16, 32, 16, "random", False), (17, 33, 17, "random", False), (31, 63, 31, "random", False),
    (32, 64, 32, "random", False), (33, 65, 33, "random", False), (35, 67, 65, "random", False),
    (17, 65, 128, "random", False), (17, 1, 128, "random", False), (17, 33, 17, "random", True),
    (17, 65, 1, "rising", False), (17, 65, 1, "falling", False), (17, 129, 1, "alternating", False),
    (17, 65, 1, "late-extreme", False), (17, 33, 1, "negative", False), (17, 33, 17, "zeros", False),
    (17, 33, 17, "uniform", False), (17, 33, 17, "zero-v", False), (17, 65, 17, "constant-v", False),
    (2, 32, 17, "cancellation", False), (17, 33, 1, "large-dot", False), (3, 2051, 17, "random", False),
    (1, 4097, 128, "uniform", False),
]


@pytest.fixture(scope="module")
def torch_stream(cuda):
    import torch

    return torch.cuda.Stream()


def _stream(default_stream: bool, torch_stream):
    return None if default_stream else torch_stream


# Every case runs with O at a 4-byte offset (the element-wise path) and, where
# d % 16 == 0, again with O 16-byte aligned (the 16-byte vector path with LDS
# DMA tile loads). K and V are followed by 64 NaN rows inside their
# allocation, so a read past row N - 1 shows up as NaN in O.
DENSE_RUNS = [(c, aligned) for c in DENSE_CASES for aligned in (False, True) if not aligned or c[2] % 16 == 0]


def _dense_id(run):
    (m, n, d, pattern, default), aligned = run
    return f"{m}x{n}x{d}-{pattern}{'-default' if default else ''}{'-aligned' if aligned else ''}"


@pytest.mark.parametrize("run", DENSE_RUNS, ids=[_dense_id(r) for r in DENSE_RUNS])
def test_dense_case(tm, oracle_lib, cuda, torch_stream, run):
    import torch

    (m, n, d, pattern, default_stream), aligned = run
    lead = 4 if aligned else 1
    q, k, v = oracle_lib.make_inputs(m, n, d, pattern)
    expected = oracle_lib.attention(q, k, v)
    dq = dev_half(q)
    dk, dv = dev_half(nan_padded_rows(k.reshape(n, d))), dev_half(nan_padded_rows(v.reshape(n, d)))
    out = guarded_lead(m * d, np.float32, GUARD_F32, fill=np.nan, lead=lead)
    stream = _stream(default_stream, torch_stream)
    print(f"dense case M={m} N={n} d={d} pattern={pattern} aligned={aligned}", flush=True)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))  # 1.0f / std::sqrt(float(d))
    code = tm.launch_fused_fp16_attention(dq, dk, dv, out.data_ptr() + 4 * lead, m, n, d, scale, stream)
    assert code == tm.SUCCESS
    torch.cuda.synchronize()
    result = host(out)
    assert (result[:lead] == GUARD_F32).all() and result[-1] == GUARD_F32, "output guard overwritten"
    compare(result[lead:-1], expected, 1e-5, 1e-4, f"TileMix vs fp64 M={m} N={n} d={d} {pattern}")
    assert np.array_equal(host(dq), q), "kernel modified the Q input"
    for device_tensor, original in ((dk, k), (dv, v)):
        assert np.array_equal(host(device_tensor).reshape(-1)[: n * d], original.reshape(-1)), \
            "kernel modified a K/V input"


def test_score_scale_reuse(tm, cuda, torch_stream):
    """Analytic (2e^-s + 4 + 8e^s) / (e^-s + 1 + e^s), reusing device buffers (:330-355)."""
    import torch

    half = lambda values: dev_half(np.array(values, dtype=np.float16).view(np.uint16))
    dq, dk, dv = half([1.0]), half([-1.0, 0.0, 1.0]), half([2.0, 4.0, 8.0])
    out = dev(np.array([GUARD_F32, np.nan, GUARD_F32], dtype=np.float32))
    for scale in (1.0, 0.0, -1.0, 0.5):
        assert tm.launch_fused_fp16_attention(dq, dk, dv, out.data_ptr() + 4, 1, 3, 1, scale,
                                              torch_stream) == tm.SUCCESS
        torch_stream.synchronize()
        result = host(out)
        assert result[0] == GUARD_F32 and result[2] == GUARD_F32
        a, b = math.exp(-scale), math.exp(scale)
        compare(result[1:2], [(2 * a + 4 + 8 * b) / (a + 1 + b)], 1e-5, 1e-4, f"scale {scale}")


QUANT_CASES = [(129, 65, 17, "zeros"), (129, 65, 1, "rounding"), (129, 65, 3, "tiny"),
               (3, 5, 128, "max-range"), (137, 73, 31, "random"), (129, 131, 17, "block-outliers")]


def quant_inputs(oracle_lib, m, n, d, pattern):
    """Inputs of the quantizer cases (src/tests/tilemix_test.cu:369-381)."""
    q, k, _ = oracle_lib.make_inputs(m, n, d, "block-outliers" if pattern == "block-outliers" else "random")
    for values in (q, k):
        flat = values.reshape(-1)
        idx = np.arange(flat.size)
        if pattern == "zeros":
            flat[:] = 0
        elif pattern == "rounding":
            ties = np.array([127, -127, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5], dtype=np.float16).view(np.uint16)
            flat[:] = ties[idx % 8]
        elif pattern == "tiny":
            flat[:] = np.where(idx % 2 == 1, np.float16(-2.0**-24), np.float16(2.0**-24)).astype(np.float16).view(np.uint16)
        elif pattern == "max-range":
            flat[:] = np.where(idx % 2 == 1, np.float16(-65504.0), np.float16(65504.0)).astype(np.float16).view(np.uint16)
    return q, k


@pytest.mark.parametrize("m,n,d,pattern", QUANT_CASES, ids=[c[3] for c in QUANT_CASES])
def test_quantizer_case(tm, oracle_lib, cuda, torch_stream, m, n, d, pattern):
    q, k = quant_inputs(oracle_lib, m, n, d, pattern)
    q_ref, qs_ref = oracle_lib.quantize(q, 128)
    k_ref, ks_ref = oracle_lib.quantize(k, 64)
    if pattern == "rounding":
        assert list(q_ref.reshape(-1)[:8]) == [127, -127, 1, -1, 2, -2, 127, -127]
    dq, dk = dev_half(q), dev_half(k)
    q8 = guarded(q.size, np.int8, GUARD_I8)
    k8 = guarded(k.size, np.int8, GUARD_I8)
    qs = guarded(qs_ref.size, np.uint16, GUARD_SCALE)
    ks = guarded(ks_ref.size, np.uint16, GUARD_SCALE)
    print(f"quantizer case M={m} N={n} d={d} pattern={pattern}", flush=True)
    code = tm.quantize_tilemix_qk(dq, dk, q8.data_ptr() + 1, k8.data_ptr() + 1, qs.data_ptr() + 2,
                                  ks.data_ptr() + 2, m, n, d, torch_stream)
    assert code == tm.SUCCESS
    torch_stream.synchronize()
    for buf, ref, guard in ((q8, q_ref.reshape(-1), GUARD_I8), (k8, k_ref.reshape(-1), GUARD_I8),
                            (qs, qs_ref, GUARD_SCALE), (ks, ks_ref, GUARD_SCALE)):
        got = host(buf).view(ref.dtype)
        assert got[0] == guard and got[-1] == guard, "guard overwritten"
        assert np.array_equal(got[1:-1], ref), f"quantizer mismatch ({pattern})"
    assert np.array_equal(host(dq), q) and np.array_equal(host(dk), k), "quantizer modified its input"


ROUTING_SHAPES = [((35, 67, 17, "random", False), 2), ((17, 2048, 5, "random", False), 1),
                  ((17, 2049, 5, "random", False), 1), ((17, 4099, 5, "random", False), 2),
                  ((35, 163, 17, "random", False), 3), ((17, 65, 17, "random", False), INT_MAX),
                  ((17, 4097, 3, "random", False), 1), ((129, 131, 17, "block-outliers", True), 1),
                  ((17, 65, 17, "zeros", False), 2), ((17, 65, 1, "rising", False), 1),
                  ((17, 65, 1, "falling", False), 1), ((17, 129, 1, "alternating", False), 1),
                  ((17, 65, 1, "late-extreme", False), 1), ((17, 33, 128, "max-int8", False), 1)]
ROUTING_CASES = [(shape, group, pattern, True) for shape, group in ROUTING_SHAPES
                 for pattern in ("fp16", "int8-requested", "mixed")]
ROUTING_CASES += [((3, 33, d, "random", False), 1, pattern, True)
                  for d in (1, 15, 16, 17, 31, 32, 33, 48, 63, 64, 65, 80, 96, 112, 127, 128)
                  for pattern in ("fp16", "int8-requested", "mixed")]
ROUTING_CASES += [((17, 2051, 5, "random", False), 1, "implicit-fp16", True),
                  ((35, 67, 17, "random", False), 2, "mixed", False)]


def _routing_id(case):
    (m, n, d, inputs, default), group, pattern, trace = case
    g = "max" if group == INT_MAX else group
    return f"{m}x{n}x{d}-{inputs}-g{g}-{pattern}{'' if trace else '-notrace'}{'-default' if default else ''}"


ROUTING_RUNS = [(c, aligned) for c in ROUTING_CASES for aligned in (False, True)
                if not aligned or c[0][2] % 16 == 0]


@pytest.mark.parametrize("run", ROUTING_RUNS,
                         ids=[_routing_id(c) + ("-aligned" if a else "") for c, a in ROUTING_RUNS])
def test_routing_case(tm, oracle_lib, cuda, torch_stream, run):
    import torch

    case, aligned = run
    lead = 4 if aligned else 1
    (m, n, d, inputs, default_stream), group, pattern, trace = case
    query_tiles, key_tiles = (m + 15) // 16, (n + 31) // 32
    implicit = pattern == "implicit-fp16"
    words, expected_bits = reference_group_words(query_tiles, key_tiles, group, pattern)
    assert words.size == tm.routing_word_count(m, n, group), "routing layout disagrees with group packing"
    q, k, v = oracle_lib.make_inputs(m, n, d, inputs)
    q8_ref, qs_ref = oracle_lib.quantize(q, 128)
    k8_ref, ks_ref = oracle_lib.quantize(k, 64)
    stream = _stream(default_stream, torch_stream)
    dq = dev_half(q)
    # K / V with 64 NaN rows after row N - 1 (see DENSE_RUNS); quantized from the first N rows.
    dk, dv = dev_half(nan_padded_rows(k.reshape(n, d))), dev_half(nan_padded_rows(v.reshape(n, d)))
    out = guarded_lead(m * d, np.float32, GUARD_F32, fill=np.nan, lead=lead)
    mask = dev(words)
    bits = guarded(expected_bits.size, np.uint8, GUARD_TRACE)
    q8 = torch.empty(q.size, dtype=torch.int8, device="cuda:0")
    k8 = torch.empty(k.size, dtype=torch.int8, device="cuda:0")
    q_scales = torch.empty(qs_ref.size, dtype=torch.int16, device="cuda:0")
    k_scales = torch.empty(ks_ref.size, dtype=torch.int16, device="cuda:0")
    dots = guarded(m * n, np.int32, GUARD_DOT)
    print(f"routing case M={m} N={n} d={d} g={group} pattern={pattern} trace={trace} aligned={aligned}",
          flush=True)
    assert tm.quantize_tilemix_qk(dq, dk, q8, k8, q_scales, k_scales, m, n, d, stream) == tm.SUCCESS
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    # All-FP16 masks must preserve the un-routed result exactly (:490-509).
    assert tm.launch_fused_fp16_attention(dq, dk, dv, out.data_ptr() + 4 * lead, m, n, d, scale,
                                          stream) == tm.SUCCESS
    torch.cuda.synchronize()
    baseline = host(out)
    routing = tm.TileMixRouting(None if implicit else mask, 0 if implicit else words.size, group,
                                bits.data_ptr() + 1 if trace else None)
    quantized = tm.TileMixQuantized(q8, k8, q_scales, k_scales, dots.data_ptr() + 4)
    assert tm.launch_fused_fp16_attention(dq, dk, dv, out.data_ptr() + 4 * lead, m, n, d, scale, stream,
                                          routing, quantized) == tm.SUCCESS
    torch.cuda.synchronize()
    actual = host(out)
    assert (actual[:lead] == GUARD_F32).all() and actual[-1] == GUARD_F32, "routed output guard overwritten"
    if not expected_bits.any():
        assert np.array_equal(actual.view(np.uint32), baseline.view(np.uint32)), \
            "all-FP16 routing changed baseline outputs"
    got_dots = host(dots)
    assert got_dots[0] == GUARD_DOT and got_dots[-1] == GUARD_DOT, "INT32 dot guard overwritten"
    cell_bits = np.repeat(np.repeat(expected_bits, 16, axis=0)[:m], 32, axis=1)[:, :n].astype(bool)
    exact = q8_ref.astype(np.int64) @ k8_ref.astype(np.int64).T
    expected_dots = np.where(cell_bits, exact, int(GUARD_DOT)).astype(np.int32)
    mismatch = got_dots[1:-1].reshape(m, n) != expected_dots
    assert not mismatch.any(), f"INT32 dot mismatch at {np.argwhere(mismatch)[:4].tolist()}"
    got_bits = host(bits)
    assert got_bits[0] == GUARD_TRACE and got_bits[-1] == GUARD_TRACE, "routing trace guard overwritten"
    want_bits = expected_bits.reshape(-1) if trace else np.full(expected_bits.size, GUARD_TRACE, np.uint8)
    assert np.array_equal(got_bits[1:-1], want_bits), "device routing-bit decoding failed"
    assert np.array_equal(host(mask).view(np.uint64), words), "routing mask modified by kernel"
    assert np.array_equal(host(q8), q8_ref.reshape(-1)) and np.array_equal(host(k8), k8_ref.reshape(-1))
    assert np.array_equal(host(q_scales).view(np.uint16), qs_ref)
    assert np.array_equal(host(k_scales).view(np.uint16), ks_ref)
    mixed = oracle_lib.tilemix(q, k, v, q8_ref, k8_ref, qs_ref, ks_ref, expected_bits, scale)
    compare(actual[lead:-1], mixed, 1e-5, 1e-4, "mixed FP16/INT8 vs fp64 TileMix oracle")
