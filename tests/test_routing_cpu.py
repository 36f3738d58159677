"""CPU checks of the host restatement used to test the device mask producer
(tests/routing_reference.py): splitmix64 against its published known answer,
the draw's range and balance, and the builders' deterministic rules against
tilemix.routing's host builders.
"""
from __future__ import annotations

import numpy as np

import routing_reference as ref
from tilemix import routing


def test_splitmix64_known_answer():
    # First output of splitmix64 from state 0 (Vigna's reference splitmix64.c).
    assert int(ref.splitmix64(0)) == 0xE220A8397B1DCDAF
    # The state advances by the golden gamma per call: output k is mix((k + 1) * gamma).
    with np.errstate(over="ignore"):
        states = np.arange(3, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15)
    outputs = ref.splitmix64(states)
    assert int(outputs[0]) == 0xE220A8397B1DCDAF
    assert len(set(int(x) for x in outputs)) == 3


def test_uniform24_range_and_balance():
    u = ref.uniform24(12345, np.arange(1 << 16, dtype=np.uint64), 0)
    assert u.dtype == np.float32 and u.min() >= 0.0 and u.max() < 1.0
    assert abs(float(u.mean()) - 0.5) < 0.01
    # 24-bit values are exact in fp32
    assert np.array_equal(u * np.float32(1 << 24), np.floor(u * np.float32(1 << 24)))
    v = ref.uniform24(12345, np.arange(1 << 16, dtype=np.uint64), 1)
    assert not np.array_equal(u, v)


def test_causal_band_rules_match_host_builder():
    S, tr, tk, band = 4096, 128, 64, 8
    codes = ref.causal_band(2, S, tr, tk, band, 0.5, seed=7)
    host = routing.causal_near_diagonal(np.random.default_rng(0), S, tr, tk, band, 0.5)[:: tr // 16, :: tk // 32]
    # skip and forced-FP16 tiles are deterministic; only the random tiles differ
    for h in range(2):
        det = (host == routing.SKIP) | (codes[h] == routing.SKIP)
        assert np.array_equal(codes[h][det], host[det])
        band_mask = np.zeros_like(det)
        tq = S // tr
        for i in range(tq):
            last = (i * tr + tr - 1) // tk
            band_mask[i, max(0, last - band + 1): last + 1] = True
        assert (codes[h][band_mask] == routing.FP16).all()
        assert (host[band_mask] == routing.FP16).all()
        rand = ~det & ~band_mask
        frac = float((codes[h][rand] == routing.INT8).mean())
        assert 0.45 < frac < 0.55


def test_three_way_rows_never_all_skipped():
    codes = ref.three_way(3, 1024, 512, 64, 64, 0.9, 0.05, seed=3)  # many all-skip rows before the fix-up
    assert not (codes == routing.SKIP).all(axis=2).any()
    raw = ref.uniform24(3, ref.linear_index(3, 16, 8), 0) < np.float32(0.9)
    assert raw.all(axis=2).any()  # the fix-up was exercised


def test_bernoulli_fraction():
    codes = ref.bernoulli(4, 2048, 2048, 64, 64, 0.25, seed=11)
    assert abs(float(codes.mean()) - 0.25) < 0.02
