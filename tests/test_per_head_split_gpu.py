"""The per-head entry point's key-range split (launch_fused_fp16_attention on a
head too small to fill the GPU: several workgroups per 128-row block, each over
a range of key tiles, partial row states merged by a combine kernel through the
library's fixed device workspace).

* Calls alternating between two streams with no synchronisation in between
  share the workspace only one at a time (the library orders split calls on a
  device through one event): every head equals the fp64 TileMix oracle.
* Ragged shapes and both O alignments (vector / element-wise combine) against
  the oracle, with the routing trace and INT32 dots exact; two of them have
  more splits than the combine takes in one batch (64 and 47).
* A call made while its stream is captured into a graph takes the plain launch
  (no workspace, no event): every replay equals the first, and the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import GUARD_DOT, GUARD_F32, GUARD_TRACE, compare, dev, dev_half, guarded, guarded_lead, host, \
    reference_group_words

pytestmark = pytest.mark.gpu


def _head(oracle_lib, m, n, d, pattern, group=2):
    q, k, v = oracle_lib.make_inputs(m, n, d, pattern)
    words, bits = reference_group_words((m + 15) // 16, (n + 31) // 32, group, "mixed")
    q8, qs = oracle_lib.quantize(q, 128)
    k8, ks = oracle_lib.quantize(k, 64)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    expected = oracle_lib.tilemix(q, k, v, q8, k8, qs, ks, bits, scale)
    return dict(q=q, k=k, v=v, words=words, bits=bits, q8=q8, k8=k8, qs=qs, ks=ks, scale=scale, expected=expected,
                m=m, n=n, d=d, group=group)


def _device(tm, h, lead=4):
    import torch

    m, n, d = h["m"], h["n"], h["d"]
    b = dict(q=dev_half(h["q"]), k=dev_half(h["k"]), v=dev_half(h["v"]), words=dev(h["words"]),
             q8=torch.empty(m * d, dtype=torch.int8, device="cuda:0"),
             k8=torch.empty(n * d, dtype=torch.int8, device="cuda:0"),
             qs=torch.empty(h["qs"].size, dtype=torch.int16, device="cuda:0"),
             ks=torch.empty(h["ks"].size, dtype=torch.int16, device="cuda:0"),
             out=guarded_lead(m * d, np.float32, GUARD_F32, fill=np.nan, lead=lead),
             trace=guarded(h["bits"].size, np.uint8, GUARD_TRACE),
             dots=guarded(m * n, np.int32, GUARD_DOT), lead=lead)
    return b


def _call(tm, h, b, stream, with_outputs=True):
    m, n, d = h["m"], h["n"], h["d"]
    tm.check(tm.quantize_tilemix_qk(b["q"], b["k"], b["q8"], b["k8"], b["qs"], b["ks"], m, n, d, stream),
             "quantize_tilemix_qk")
    routing = tm.TileMixRouting(b["words"], h["words"].size, h["group"],
                                b["trace"].data_ptr() + 1 if with_outputs else None)
    quantized = tm.TileMixQuantized(b["q8"], b["k8"], b["qs"], b["ks"],
                                    b["dots"].data_ptr() + 4 if with_outputs else None)
    tm.check(tm.launch_fused_fp16_attention(b["q"], b["k"], b["v"], b["out"].data_ptr() + 4 * b["lead"], m, n, d,
                                            h["scale"], stream, routing, quantized), "launch_fused_fp16_attention")


def _check(h, b, exact_outputs=True):
    lead = b["lead"]
    actual = host(b["out"])
    assert (actual[:lead] == GUARD_F32).all() and actual[-1] == GUARD_F32, "output guard overwritten"
    compare(actual[lead:-1], h["expected"], 1e-5, 1e-4, "split per-head call vs fp64 TileMix oracle")
    if not exact_outputs:
        return
    bits = host(b["trace"])
    assert bits[0] == GUARD_TRACE and bits[-1] == GUARD_TRACE
    assert np.array_equal(bits[1:-1], h["bits"].reshape(-1)), "routing trace"
    m, n = h["m"], h["n"]
    cells = np.repeat(np.repeat(h["bits"], 16, axis=0)[:m], 32, axis=1)[:, :n].astype(bool)
    exact = (h["q8"].astype(np.float64) @ h["k8"].astype(np.float64).T).astype(np.int64)
    want = np.where(cells, exact, int(GUARD_DOT)).astype(np.int32)
    dots = host(b["dots"])
    assert dots[0] == GUARD_DOT and dots[-1] == GUARD_DOT
    assert np.array_equal(dots[1:-1].reshape(m, n), want), "INT32 dots"


def test_split_calls_on_two_streams(tm, oracle_lib, cuda):
    import torch

    heads = [_head(oracle_lib, 2048, 2048, 128, "random"), _head(oracle_lib, 1536, 3000, 64, "random"),
             _head(oracle_lib, 2048, 2048, 128, "block-outliers"), _head(oracle_lib, 1024, 4096, 128, "random")]
    buffers = [_device(tm, h) for h in heads]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    print("split per-head calls on two streams", flush=True)
    for i, (h, b) in enumerate(zip(heads, buffers)):
        _call(tm, h, b, streams[i % 2])
    torch.cuda.synchronize()
    for h, b in zip(heads, buffers):
        _check(h, b)


@pytest.mark.parametrize("m,n,d,lead", [(1000, 2500, 128, 4), (1000, 2500, 128, 1), (777, 3001, 48, 4),
                                        (512, 1024, 32, 4), (128, 8192, 128, 4), (300, 6000, 64, 1)],
                         ids=["ragged-vector", "ragged-scalar", "d48", "small",
                              "64-splits", "47-splits-scalar"])
def test_split_ragged_shapes(tm, oracle_lib, cuda, m, n, d, lead):
    import torch

    h = _head(oracle_lib, m, n, d, "random", group=3)
    b = _device(tm, h, lead=lead)
    print(f"split per-head call M={m} N={n} d={d} lead={lead}", flush=True)
    _call(tm, h, b, None)
    torch.cuda.synchronize()
    _check(h, b)


def test_per_head_call_under_graph_capture(tm, oracle_lib, cuda):
    import torch

    h = _head(oracle_lib, 2048, 2048, 128, "random")
    b = _device(tm, h)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        _call(tm, h, b, side, with_outputs=False)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print("per-head call under graph capture", flush=True)
    with torch.cuda.graph(graph):
        _call(tm, h, b, torch.cuda.current_stream(), with_outputs=False)
    torch.cuda.synchronize()
    first = None
    for replay in range(3):
        b["out"][b["lead"]:-1].fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = host(b["out"]).copy()
        if first is None:
            first = got
        assert np.array_equal(got.view(np.int32), first.view(np.int32)), f"replay {replay} differs"
        _check(h, b, exact_outputs=False)
