"""Host logic on the CPU: routing-word packing, the sizing helpers, the
BASELINE routing-mask builders and the algorithmic work model.

Packing is checked against the independent group packer of
src/tests/tilemix_test.cu:432-448 (restated in tests/helpers.py) and against
the oracle's decoder; the sizing helpers against the known values the
reference's own tests hold (src/tests/tilemix_test.cu:186-217).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
from helpers import reference_group_words
from tilemix import routing, workloads

INT_MAX = 2 ** 31 - 1


def test_word_count_known_values():
    # src/tests/tilemix_test.cu:208-217
    assert routing.word_count(17, 2048, 1) == 2
    assert routing.word_count(17, 2049, 1) == 4
    assert routing.word_count(17, 4097, 2) == 4
    assert routing.word_count(17, 4097, 1) == 6
    assert routing.word_count(17, INT_MAX, INT_MAX) == 2
    assert routing.word_count(0, 1, 1) == 0
    assert routing.word_count(1, 0, 1) == 0
    assert routing.word_count(1, 1, 0) == 0


@pytest.mark.parametrize("m,n,g", [(1, 1, 1), (17, 2049, 1), (40, 4097, 2), (100, 9000, 5), (16, 64 * 32 * 3, 1),
                                   (4096, 4096, 2), (16384, 16384, 2)])
def test_word_count_matches_independent_packer(m, n, g):
    qt, kt = (m + 15) // 16, (n + 31) // 32
    if qt * kt > 2_000_000:
        groups = (kt + g - 1) // g
        assert routing.word_count(m, n, g) == qt * ((groups + 63) // 64)
        return
    words, _ = reference_group_words(qt, kt, g, "mixed")
    assert routing.word_count(m, n, g) == words.size


@pytest.mark.parametrize("m,n,g", [(17, 2049, 1), (40, 4097, 2), (33, 700, 3), (256, 256, 2), (48, 64 * 32 * 2 + 5, 2)])
def test_pack_cells_round_trip(m, n, g):
    qt, kt = (m + 15) // 16, (n + 31) // 32
    _, bits = reference_group_words(qt, kt, g, "mixed")
    _, skip_bits = reference_group_words(qt, kt, g, "int8-requested")
    rng = np.random.default_rng(m + n)
    codes = bits.astype(np.uint8)
    # mark a random set of whole groups as skipped
    groups = (kt + g - 1) // g
    skip_groups = rng.random((qt, groups)) < 0.3
    skip = np.repeat(skip_groups, g, axis=1)[:, :kt]
    codes = np.where(skip, routing.SKIP, codes).astype(np.uint8)
    route_words, skip_words = routing.pack_cells(codes, g)
    assert route_words.size == routing.word_count(m, n, g)
    decoded = oracle.decode_routes(route_words, skip_words, m, n, g)
    assert np.array_equal(decoded, codes)
    # INT8 bits of the packed words agree with the independent packer where not skipped
    words_ref, _ = reference_group_words(qt, kt, g, "mixed")
    decoded_plain = oracle.decode_routes(words_ref, None, m, n, g)
    assert np.array_equal(decoded_plain[~skip], codes[~skip])


def test_pack_cells_rejects_non_uniform_groups():
    codes = np.zeros((2, 4), dtype=np.uint8)
    codes[0, 1] = routing.INT8
    with pytest.raises(ValueError):
        routing.pack_cells(codes, 2)


def test_cells_from_tiles_replication():
    tiles = np.array([[0, 1, 2], [1, 0, 1]], dtype=np.uint8)
    cells = routing.cells_from_tiles(tiles, 64, 64, 100, 150)
    assert cells.shape == (7, 5)
    assert np.array_equal(cells[:4, :2], np.zeros((4, 2)))
    assert np.array_equal(cells[:4, 2:4], np.ones((4, 2)))
    assert (cells[:4, 4] == 2).all() and (cells[4:, 4] == 1).all()
    with pytest.raises(ValueError):
        routing.cells_from_tiles(tiles, 24, 64, 100, 150)


def test_causal_band_builder_matches_spec():
    # Config 3: 128x64 tiles; key tile j of query tile i is above the diagonal
    # when j >= 2i + 2 (skipped); the 8 tiles with (2i + 1) - j < 8 are FP16;
    # the rest are INT8 with p = 0.5. Per head 1056 tiles run, 244 forced FP16.
    S = 4096
    codes = routing.causal_near_diagonal(np.random.default_rng(0), S, 128, 64)
    tiles = codes[::8, ::2]
    i = np.arange(32)[:, None]
    j = np.arange(64)[None, :]
    assert np.array_equal(tiles == routing.SKIP, j >= 2 * i + 2)
    visible = j < 2 * i + 2
    forced = visible & ((2 * i + 1) - j < 8)
    assert (tiles[forced] == routing.FP16).all()
    assert int(visible.sum()) == 1056 and int(forced.sum()) == 244
    free = visible & ~forced
    assert int(free.sum()) == 812
    frac = (tiles[free] == routing.INT8).mean()
    assert 0.4 < frac < 0.6
    # replicated over cells: every cell of a tile carries the tile's code
    assert np.array_equal(codes, routing.cells_from_tiles(tiles, 128, 64, S, S))


def test_importance_router_top_quarter():
    rng = np.random.default_rng(1)
    qa = rng.random(8)
    ka = rng.random(16)
    ka[3] = ka[4]  # a tie, broken by tile index
    codes = routing.importance_top_fraction(qa, ka, 1024, 1024, 128, 128, 64)
    tiles = codes[::8, ::2]
    est = 128 * np.outer(qa, ka)
    fp16 = tiles == routing.FP16
    assert int(fp16.sum()) == 32
    assert est[fp16].min() >= est[~fp16].max()


def test_three_way_builder():
    codes = routing.three_way(np.random.default_rng(2), 8192, 8192, 64, 64)
    tiles = codes[::4, ::2]
    fr = [(tiles == c).mean() for c in (routing.SKIP, routing.INT8, routing.FP16)]
    assert abs(fr[0] - 0.3) < 0.02 and abs(fr[1] - 0.4) < 0.02 and abs(fr[2] - 0.3) < 0.02
    assert (tiles != routing.SKIP).any(axis=1).all()
    small = routing.three_way(np.random.default_rng(3), 128, 128, 64, 64, p_skip=0.999, p_int8=0.0)
    assert (small != routing.SKIP).any(axis=1).all()


def brute_pairs(codes, M, N, causal):
    counts = {0: 0, 1: 0, 2: 0}
    for qi in range(M):
        for kj in range(N):
            if causal and kj > qi:
                continue
            counts[int(codes[qi // 16, kj // 32])] += 1
    return {"fp16": counts[0], "int8": counts[1], "skip": counts[2]}


@pytest.mark.parametrize("M,N,causal", [(50, 70, False), (96, 96, True), (130, 130, True), (33, 200, False)])
def test_pair_counts_brute_force(M, N, causal):
    rng = np.random.default_rng(M + N)
    codes = rng.integers(0, 3, size=((M + 15) // 16, (N + 31) // 32)).astype(np.uint8)
    assert routing.pair_counts(codes, M, N, causal) == brute_pairs(codes, M, N, causal)


def test_causal_headline_work_closed_form():
    # Causal count is S(S+1)/2 visible pairs per head; above-diagonal skip tiles hold none.
    S, D = 4096, 128
    codes = routing.causal_near_diagonal(np.random.default_rng(0), S, 128, 64)
    pairs = routing.pair_counts(codes, S, S, True)
    assert pairs["int8"] + pairs["fp16"] == S * (S + 1) // 2 and pairs["skip"] == 0
    work = routing.algorithmic_work(codes, S, S, D, True)
    assert work["ops_int8"] == 2 * D * pairs["int8"]
    assert work["flops_fp16"] == 2 * D * pairs["fp16"] + 2 * D * (S * (S + 1) // 2)


def test_workload_table():
    w3 = workloads.WORKLOADS[3]
    assert (w3.B, w3.H, w3.S, w3.D, w3.causal, w3.heads) == (4, 16, 4096, 128, True, 64)
    assert w3.score_scale == float(np.float32(1) / np.sqrt(np.float32(128)))
    assert [workloads.WORKLOADS[i].heads for i in range(1, 6)] == [4, 64, 64, 32, 32]
    for w in workloads.WORKLOADS.values():
        assert w.S % 128 == 0 and w.D in (64, 128)
        assert math.isclose(w.score_scale, 1 / math.sqrt(w.D), rel_tol=1e-7)


def test_pack_heads_concatenates_per_head_words():
    w = workloads.WORKLOADS[1]
    codes = workloads.make_codes(w, 7)
    assert codes.shape == (4, 16, 8)
    route, skip = workloads.pack_heads(codes, w.key_tiles_per_group)
    per_head = routing.word_count(w.S, w.S, w.key_tiles_per_group)
    assert skip is None and route.size == 4 * per_head
    for h in range(4):
        decoded = oracle.decode_routes(route[h * per_head:(h + 1) * per_head], None, w.S, w.S, 2)
        assert np.array_equal(decoded, codes[h])


def test_bench_refuses_more_than_one_gpu():
    """bench.py is a one-GPU benchmark: --gpus N > 1 exits with code 2 and a
    JSON line naming the reason, before touching any device."""
    import json
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    proc = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120, cwd=root)
    assert proc.returncode == 2, proc.stderr
    line = json.loads(proc.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def _bench_module():
    import importlib.util
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    spec = importlib.util.spec_from_file_location("bench_module", root / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    return bench


def test_bench_parses_the_dpm_sclk_sysfs_file():
    """bench.py reads the shader clock from the card's `pp_dpm_sclk` file, whose level
    in use is marked with '*' (amdgpu sysfs layout), and returns None for a file with no
    marked level rather than a wrong number."""
    bench = _bench_module()
    assert bench.parse_dpm_sclk("0: 500Mhz\n1: 2040Mhz *\n2: 2400Mhz\n") == 2040.0
    assert bench.parse_dpm_sclk("0: 500Mhz *\n1: 2400Mhz\n") == 500.0
    assert bench.parse_dpm_sclk("0: 500Mhz\n1: 2400Mhz\n") is None
    assert bench.parse_dpm_sclk("S: *\n") is None
    assert bench.parse_dpm_sclk("") is None


def test_bench_clock_sampler_starts_no_process(tmp_path, monkeypatch):
    """The clock sampler runs inside the process that drives the GPU, so it must never
    start another program: under rocprofv3 the profiler's preloaded library would
    come along and the child's exec would happen from a GPU-initialised process. Every
    way of starting a process is patched to raise; the sampler still returns the clock
    from a sysfs-layout file (and None when the file is missing), and the steps it ran."""
    import os
    import subprocess

    bench = _bench_module()
    started = []

    def refuse(*args, **kwargs):
        started.append(args)
        raise AssertionError("the clock sampler started a process")

    monkeypatch.setattr(subprocess, "Popen", refuse)
    monkeypatch.setattr(subprocess, "run", refuse)
    for name in ("system", "fork", "posix_spawn", "posix_spawnp", "execv", "execve", "execvp", "execvpe",
                 "spawnv", "spawnve", "popen"):
        if hasattr(os, name):
            monkeypatch.setattr(os, name, refuse)

    sysfs = tmp_path / "pp_dpm_sclk"
    sysfs.write_text("0: 500Mhz\n1: 2105Mhz *\n2: 2400Mhz\n")
    steps = []
    mhz, ran = bench.sample_sclk_mhz(lambda: steps.append(1), lambda: None, files=[sysfs], reads=3)
    assert mhz == 2105.0
    assert ran == len(steps) and ran > 0
    mhz, _ = bench.sample_sclk_mhz(lambda: None, lambda: None, files=[tmp_path / "missing"], reads=3)
    assert mhz is None
    mhz, _ = bench.sample_sclk_mhz(lambda: None, lambda: None, files=[], reads=3)
    assert mhz is None
    assert started == []
