"""Whole-tile skip patterns against the C oracle, through the C ABI.

The attention kernel steps over a 64-key tile whose cells are all skipped
for the workgroup's 128 rows, and alternates its two V buffers per visited
tile, so the buffer a tile lands in depends on how many tiles were skipped
before it. These cases skip whole tiles in fixed patterns (every other tile,
runs of two and three, all but the first, all but the last, a skipped first
tile) with random INT8 / FP16 routes on the visible tiles, on the vector
path (16-byte aligned O) and the element-wise path (O at a 4-byte offset),
causal and not. Outputs must be within max-abs 2e-3 / mean-abs 2e-4 of the
fp64 oracle (src/tests/reference_tilemix.h restated in oracle/), with the
quantized operands and scales bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import GUARD_F32, dev, dev_half, guarded_lead, host

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-3, 2e-4
M, N, D, G = 256, 1024, 128, 2  # 2 query workgroups, 16 key tiles of 64, one routing group per tile

PATTERNS = {
    "alternate": [t % 2 == 1 for t in range(16)],
    "runs": [t in (1, 2, 5, 6, 7, 10) for t in range(16)],
    "only-first": [t != 0 for t in range(16)],
    "only-last": [t != 15 for t in range(16)],
    "first-skipped": [t in (0, 3) for t in range(16)],
}


def f16_bits(t) -> np.ndarray:
    import torch

    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("aligned", [True, False], ids=["vector", "elementwise"])
@pytest.mark.parametrize("causal", [False, True], ids=["dense", "causal"])
@pytest.mark.parametrize("pattern", list(PATTERNS))
def test_whole_tile_skip_patterns(tm, oracle_lib, cuda, pattern, causal, aligned):
    import torch

    from tilemix import routing

    rng = np.random.default_rng(sum(map(ord, pattern)) + 2 * causal + aligned)
    q = oracle_lib.float_to_half(rng.standard_normal((M, D)).astype(np.float32))
    k = oracle_lib.float_to_half(rng.standard_normal((N, D)).astype(np.float32))
    v = oracle_lib.float_to_half(rng.standard_normal((N, D)).astype(np.float32))
    # Cells are 16 rows x 32 keys; a 64-key tile is two cells wide and one
    # routing group (G = 2), so codes are drawn per (16-row block, tile).
    tiles = rng.integers(0, 2, size=(M // 16, N // 64)).astype(np.uint8)  # 0 FP16, 1 INT8
    for t, skipped in enumerate(PATTERNS[pattern]):
        if skipped:
            tiles[:, t] = routing.SKIP
    if causal:
        # A row block whose visible tiles are all skipped would keep no key:
        # give it an FP16 diagonal tile.
        for r in range(M // 16):
            diagonal = (16 * r) // 64
            if (tiles[r, :diagonal + 1] == routing.SKIP).all():
                tiles[r, diagonal] = 0
    codes = np.repeat(tiles, 2, axis=1)
    route, skip = routing.pack_cells(codes, G)
    lead = 4 if aligned else 1
    O = guarded_lead(M * D, np.float32, GUARD_F32, fill=np.float32(777.0), lead=lead)
    Q8 = torch.empty((M, D), dtype=torch.int8, device="cuda:0")
    K8 = torch.empty((N, D), dtype=torch.int8, device="cuda:0")
    qs = torch.empty(((M + 127) // 128,), dtype=torch.int16, device="cuda:0")
    ks = torch.empty(((N + 63) // 64,), dtype=torch.int16, device="cuda:0")
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    args = tm.BatchedArgs(Q=dev_half(q), K=dev_half(k), V=dev_half(v), O=O.data_ptr() + 4 * lead, heads=1, M=M, N=N,
                          d=D, score_scale=scale, causal=causal, quantize=1, route_words=dev(route),
                          skip_words=dev(skip), key_tiles_per_group=G, Q8=Q8, K8=K8, q_scales=qs, k_scales=ks)
    print(f"tile skip pattern={pattern} causal={causal} aligned={aligned}", flush=True)
    tm.check(tm.attention_batched(args))
    torch.cuda.synchronize()
    out = host(O)
    assert (out[:lead] == GUARD_F32).all() and out[-1] == GUARD_F32, "output guard overwritten"
    got = out[lead:-1].reshape(M, D)
    q8_ref, qs_ref = oracle_lib.quantize(q, 128)
    k8_ref, ks_ref = oracle_lib.quantize(k, 64)
    assert np.array_equal(Q8.cpu().numpy(), q8_ref) and np.array_equal(K8.cpu().numpy(), k8_ref)
    assert np.array_equal(f16_bits(qs), qs_ref) and np.array_equal(f16_bits(ks), ks_ref)
    expected = oracle_lib.tilemix(q, k, v, q8_ref, k8_ref, qs_ref, ks_ref, codes, scale, causal)
    assert np.isfinite(got).all()
    err = np.abs(got.astype(np.float64) - expected)
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (float(err.max()), float(err.mean()))
