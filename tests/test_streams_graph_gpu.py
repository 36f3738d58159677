"""Stream ordering and graph capture of the bindings, through the C ABI.

* tilemix_tiles_importance_noalloc captured in a CUDA graph replays to the
  workspace entry point's tile codes (in this process, after an eager call),
  and also when the process's first noalloc call is made inside the capture
  (a fresh child process, tests/noalloc_capture_child.py).
* stream=None means torch's current stream: inputs produced on a side stream
  and consumed by bindings called with stream=None inside
  `with torch.cuda.stream(side)` without a synchronisation in between give the
  results of explicitly-streamed calls after a full synchronisation.
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from tilemix import routing

pytestmark = pytest.mark.gpu
HERE = Path(__file__).resolve().parent


def _router_inputs(torch, heads, M, N, d, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    q = torch.randn(heads, M, d, generator=g, device="cuda")
    k = torch.randn(heads, N, d, generator=g, device="cuda")
    q[..., :2] *= 8.0
    k[..., :2] *= 8.0
    return q.half().contiguous(), k.half().contiguous()


def test_noalloc_router_replays_in_a_graph(tm, cuda):
    import torch

    heads, M, N, d, tr, tk, fraction = 3, 2048, 1024, 128, 128, 64, 0.25
    print(f"noalloc graph: heads={heads} M={M} N={N} d={d} tile={tr}x{tk}", flush=True)
    q, k = _router_inputs(torch, heads, M, N, d, 5)
    tiles = (heads, M // tr, N // tk)
    need = tm.importance_workspace_bytes(heads, M, N, tr, tk)
    ws = torch.empty(need // 4, dtype=torch.float32, device="cuda")
    expected = torch.full(tiles, 0xEE, dtype=torch.uint8, device="cuda")
    tm.check(tm.tiles_importance(q, k, heads, M, N, d, tr, tk, fraction, ws, need, expected), "importance")
    codes = torch.full(tiles, 0xEE, dtype=torch.uint8, device="cuda")
    tm.check(tm.tiles_importance_noalloc(q, k, heads, M, N, d, tr, tk, fraction, codes), "eager noalloc")
    torch.cuda.synchronize()
    assert torch.equal(codes, expected)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = tm.tiles_importance_noalloc(q, k, heads, M, N, d, tr, tk, fraction, codes)
    tm.check(rc, "noalloc under capture")
    torch.cuda.synchronize()
    for replay in range(4):
        codes.fill_(0xEE)  # eager work between replays
        torch.cuda.synchronize()
        print(f"noalloc graph: replay {replay}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(codes, expected), f"replay {replay}"


def test_noalloc_first_call_inside_capture(cuda):
    """The scratch-address lookup of the first noalloc call on a device happens
    inside the capture: run in a fresh process so that it really is the first."""
    print("noalloc capture: child process", flush=True)
    result = subprocess.run([sys.executable, str(HERE / "noalloc_capture_child.py")], capture_output=True, text=True,
                            timeout=110)
    print(result.stdout[-2000:], result.stderr[-2000:], flush=True)
    assert result.returncode == 0
    assert result.stdout.strip().endswith("OK")


def test_default_stream_follows_torch_current_stream(tm, cuda):
    import torch

    heads, S, d = 4, 1024, 128
    print(f"current stream: heads={heads} S={S} d={d}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    src = [torch.randn(heads, S, d, generator=g, device="cuda").half() for _ in range(3)]
    rng = np.random.default_rng(4)
    words = np.concatenate([routing.pack_cells(routing.bernoulli_tiles(rng, S, S, 64, 64, 0.5), 2)[0]
                            for _ in range(heads)])
    route = torch.from_numpy(words.view(np.int64)).cuda()
    torch.cuda.synchronize()

    def outputs():
        return dict(O=torch.full((heads, S, d), float("nan"), device="cuda"),
                    K8=torch.zeros(heads, S, d, dtype=torch.int8, device="cuda"),
                    ks=torch.zeros(heads, S // 64, dtype=torch.int16, device="cuda"))

    def call(Q, K, V, out, stream):
        tm.check(tm.quantize_tilemix_qk_batched(None, K, None, out["K8"], None, out["ks"], heads, S, S, d,
                                                stream=stream), "quantize K")
        args = tm.BatchedArgs(Q=Q, K=K, V=V, O=out["O"], heads=heads, M=S, N=S, d=d, score_scale=d ** -0.5,
                              quantize=2, route_words=route, key_tiles_per_group=2, K8=out["K8"],
                              k_scales=out["ks"])
        tm.check(tm.attention_batched(args, stream), "attention")

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    implicit = outputs()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        # Delay the producer on the side stream, then write the inputs there.
        a = torch.randn(4096, 4096, device="cuda")
        for _ in range(8):
            a = a @ a
            a = a / a.abs().amax()
        Q, K, V = (torch.empty_like(x) for x in src)
        for dst, x in zip((Q, K, V), src):
            dst.copy_(x)  # runs after the matrix products on the side stream
        call(Q, K, V, implicit, None)  # stream=None: the side stream, no sync in between
    torch.cuda.synchronize()
    explicit = outputs()
    call(src[0], src[1], src[2], explicit, torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert torch.equal(implicit["K8"], explicit["K8"])
    assert torch.equal(implicit["ks"], explicit["ks"])
    assert torch.equal(implicit["O"].view(torch.int32), explicit["O"].view(torch.int32))
