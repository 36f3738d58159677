"""Repeated-launch determinism at full BASELINE size.

The attention kernel orders its LDS tile loads by hand (inline-asm DMA that
the compiler cannot see, explicit vmcnt waits and workgroup barriers), so a
missing wait would show up as a rare, launch-dependent difference rather than
as a failed single-shot parity check. Config 3 (causal, the headline) and
config 5 (skip-heavy three-way routing) are launched back to back, with the
fused quantization on, and every launch's O, K8, Q8 and scales must equal the
first launch's bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import dev

pytestmark = pytest.mark.gpu

LAUNCHES = 10


@pytest.mark.parametrize("config", [3, 5])
def test_repeated_launches_bitwise_identical(tm, cuda, config):
    import torch

    from tilemix import workloads

    w = workloads.WORKLOADS[config]
    Q, K, V = workloads.make_inputs(w, 11)
    codes = workloads.make_codes(w, 11, Q, K)
    route_np, skip_np = workloads.pack_heads(codes, w.key_tiles_per_group)
    heads, S, D = w.heads, w.S, w.D
    O = torch.empty((heads, S, D), dtype=torch.float32, device=cuda)
    Q8 = torch.empty((heads, S, D), dtype=torch.int8, device=cuda)
    K8 = torch.empty((heads, S, D), dtype=torch.int8, device=cuda)
    qs = torch.empty((heads, (S + 127) // 128), dtype=torch.int16, device=cuda)
    ks = torch.empty((heads, (S + 63) // 64), dtype=torch.int16, device=cuda)
    args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O, heads=heads, M=S, N=S, d=D, score_scale=w.score_scale,
                          causal=w.causal, quantize=1, route_words=dev(route_np),
                          skip_words=dev(skip_np) if skip_np is not None else None,
                          key_tiles_per_group=w.key_tiles_per_group, Q8=Q8, K8=K8, q_scales=qs, k_scales=ks)
    outputs = (O, Q8, K8, qs, ks)
    names = ("O", "Q8", "K8", "q_scales", "k_scales")
    print(f"determinism {w.describe()}: launch 0", flush=True)
    tm.check(tm.attention_batched(args), "attention_batched")
    torch.cuda.synchronize()
    assert torch.isfinite(O).all(), "non-finite output"
    first = [t.clone() for t in outputs]
    for launch in range(1, LAUNCHES + 1):
        for t in outputs:
            t.zero_()  # a launch that skipped a write would leave zeros, not the last result
        tm.check(tm.attention_batched(args), "attention_batched")
        torch.cuda.synchronize()
        for name, t, ref in zip(names, outputs, first):
            same = torch.equal(t.view(torch.int8) if t.dtype != torch.int8 else t,
                               ref.view(torch.int8) if ref.dtype != torch.int8 else ref)
            assert same, f"config {config}: launch {launch} differs from launch 0 in {name}"
        print(f"determinism config {config}: launch {launch} identical", flush=True)
