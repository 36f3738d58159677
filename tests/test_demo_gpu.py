"""The reference demo's workload (src/main.cu:22-69): M = 1000 queries,
N = 1003 keys, d = 128, key tiles grouped by 2 with every routing word
0xaaaa... (odd groups INT8, even groups FP16), inputs periodic in the flat
index (periods 17, 19, 23; src/main.cu:38-40).

* Through the bindings: Q8 / K8 / scales bit-exact against the oracle
  quantizer, the routing trace equal to the mask's cells, and every row of O
  within the reference suite's 1e-5 + 1e-4|x| of the fp64 oracle.
* The native demo program (tilemix-cuda_amd/examples/demo_main.cpp, the
  reference caller restated over include/attention_fused.h): its two output
  lines in the reference's format, output[0] against the oracle, and its
  optional timed rounds.
"""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from helpers import GUARD_TRACE, compare, dev, dev_half, guarded, host

pytestmark = pytest.mark.gpu

M, N, D, GROUP = 1000, 1003, 128, 2
DEMO = Path(__file__).resolve().parent.parent / "tilemix-cuda_amd" / "_build" / "tilemix_demo"


def _demo_inputs(oracle_lib):
    """fp16 bits of Q, K, V as src/main.cu:38-40 computes them (float products, then fp16)."""
    def periodic(count, period, offset, step):
        i = np.arange(count, dtype=np.int64)
        values = np.float32(step) * ((i % period) - offset).astype(np.float32)
        return oracle_lib.float_to_half(values.astype(np.float32))
    q = periodic(M * D, 17, 8, 0.125).reshape(M, D)
    k = periodic(N * D, 19, 9, 0.125).reshape(N, D)
    v = periodic(N * D, 23, 11, 0.1).reshape(N, D)
    return q, k, v


def _demo_routes():
    """Cell (query tile, key tile) routes of the all-0xaaaa... mask: INT8 where the key tile's group is odd."""
    kt = np.arange((N + 31) // 32)
    return np.repeat(((kt // GROUP) % 2 == 1).astype(np.uint8)[None, :], (M + 15) // 16, axis=0)


@pytest.fixture(scope="module")
def expected(oracle_lib):
    q, k, v = _demo_inputs(oracle_lib)
    q8, qs = oracle_lib.quantize(q, 128)
    k8, ks = oracle_lib.quantize(k, 64)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    routes = _demo_routes()
    out = oracle_lib.tilemix(q, k, v, q8, k8, qs, ks, routes, scale)
    return dict(q=q, k=k, v=v, q8=q8, qs=qs, k8=k8, ks=ks, routes=routes, scale=scale, out=out)


def test_demo_through_bindings(tm, cuda, expected):
    import torch

    e = expected
    words = np.full(tm.routing_word_count(M, N, GROUP), 0xAAAAAAAAAAAAAAAA, dtype=np.uint64)
    Q, K, V = dev_half(e["q"]), dev_half(e["k"]), dev_half(e["v"])
    Q8 = torch.empty(M * D, dtype=torch.int8, device="cuda:0")
    K8 = torch.empty(N * D, dtype=torch.int8, device="cuda:0")
    qs = torch.empty(e["qs"].size, dtype=torch.int16, device="cuda:0")
    ks = torch.empty(e["ks"].size, dtype=torch.int16, device="cuda:0")
    O = torch.full((M * D,), float("nan"), dtype=torch.float32, device="cuda:0")
    trace = guarded(e["routes"].size, np.uint8, GUARD_TRACE)
    route = dev(words)
    print(f"reference demo through the bindings: M={M} N={N} d={D} g={GROUP}", flush=True)
    tm.check(tm.quantize_tilemix_qk(Q, K, Q8, K8, qs, ks, M, N, D, None), "quantize_tilemix_qk")
    tm.check(tm.launch_fused_fp16_attention(Q, K, V, O, M, N, D, e["scale"], None,
                                            tm.TileMixRouting(route, words.size, GROUP, trace.data_ptr() + 1),
                                            tm.TileMixQuantized(Q8, K8, qs, ks)), "launch_fused_fp16_attention")
    torch.cuda.synchronize()
    assert np.array_equal(host(Q8).reshape(M, D), e["q8"]), "Q8"
    assert np.array_equal(host(K8).reshape(N, D), e["k8"]), "K8"
    assert np.array_equal(host(qs).view(np.uint16), e["qs"]) and np.array_equal(host(ks).view(np.uint16), e["ks"])
    bits = host(trace)
    assert bits[0] == GUARD_TRACE and bits[-1] == GUARD_TRACE
    assert np.array_equal(bits[1:-1], e["routes"].reshape(-1)), "routing trace"
    compare(host(O), e["out"], 1e-5, 1e-4, "reference demo vs fp64 TileMix oracle")


def test_native_demo_program(cuda, expected):
    if not DEMO.exists():
        pytest.fail(f"{DEMO} is not built; run __graft_entry__.build()")
    print(f"native demo: {DEMO} --rounds 10", flush=True)
    out = subprocess.run([str(DEMO), "--rounds", "10"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    lines = out.stdout.splitlines()
    first = re.fullmatch(r"TileMix attention: M=1000 N=1003 d=128 output\[0\]=(\S+)", lines[0])
    assert first, lines[0]
    value, want = float(first.group(1)), float(expected["out"][0, 0])
    assert abs(value - want) <= 1e-5 + 1e-4 * abs(want), (value, want)
    groups = ((N + 31) // 32 + GROUP - 1) // GROUP
    words = (M + 15) // 16 * ((groups + 63) // 64)
    assert lines[1] == f"Routing: 2 key tiles/group, {words} packed words; bit 0=FP16, bit 1=INT8 MFMA", lines[1]
    timed = re.fullmatch(r"Timed: 10 rounds of quantize_tilemix_qk \+ launch_fused_fp16_attention, (\S+) us per round",
                         lines[2])
    assert timed and float(timed.group(1)) > 0.0, lines[2]
