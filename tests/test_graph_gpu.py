"""The batched entry points inside a captured HIP graph (torch.cuda.CUDAGraph):
the library allocates nothing, issues no memset and keeps no per-call host
state, so a captured quantize + attention step replays to the eager result.
Each replay runs between other eager work and synchronisations and is
compared with the eager outputs bit for bit (O, K8, k_scales, Q8, q_scales).
"""
from __future__ import annotations

import numpy as np
import pytest

from tilemix import routing

pytestmark = pytest.mark.gpu


def test_captured_step_replays_to_the_eager_result(tm, cuda):
    import torch

    heads, S, d = 4, 512, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    Q, K, V = (torch.randn(heads, S, d, generator=g, device="cuda").half() for _ in range(3))
    rng = np.random.default_rng(3)
    words = np.concatenate([routing.pack_cells(routing.bernoulli_tiles(rng, S, S, 64, 64, 0.5), 2)[0]
                            for _ in range(heads)])
    route = torch.from_numpy(words.view(np.int64)).cuda()

    def buffers():
        return dict(O=torch.empty(heads, S, d, device="cuda"),
                    K8=torch.empty(heads, S, d, dtype=torch.int8, device="cuda"),
                    ks=torch.empty(heads, S // 64, dtype=torch.int16, device="cuda"),
                    Q8=torch.empty(heads, S, d, dtype=torch.int8, device="cuda"),
                    qs=torch.empty(heads, S // 128, dtype=torch.int16, device="cuda"))

    def step(b, stream):
        tm.check(tm.quantize_tilemix_qk_batched(None, K, None, b["K8"], None, b["ks"], heads, S, S, d,
                                                stream=stream), "quantize K")
        args = tm.BatchedArgs(Q=Q, K=K, V=V, O=b["O"], heads=heads, M=S, N=S, d=d, score_scale=d ** -0.5,
                              causal=True, quantize=2, route_words=route, key_tiles_per_group=2,
                              K8=b["K8"], k_scales=b["ks"], Q8=b["Q8"], q_scales=b["qs"])
        tm.check(tm.attention_batched(args, stream), "attention")

    print("graph capture: eager reference", flush=True)
    eager = buffers()
    step(eager, torch.cuda.current_stream())
    torch.cuda.synchronize()

    captured = buffers()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # warm-up launch outside the capture
        step(captured, stream)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print("graph capture: capturing", flush=True)
    with torch.cuda.graph(graph):
        step(captured, torch.cuda.current_stream())
    torch.cuda.synchronize()
    for replay in range(4):
        for t in captured.values():
            t.fill_(0 if t.dtype != torch.float32 else float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        print(f"graph capture: replay {replay}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        for name in eager:
            a, b = eager[name], captured[name]
            if a.dtype == torch.float32:
                a, b = a.view(torch.int32), b.view(torch.int32)
            assert torch.equal(a, b), f"replay {replay}: {name}"
