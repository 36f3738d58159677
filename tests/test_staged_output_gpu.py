"""The batched entry point's LDS-staged O stores (fp32 O, d = 128 or 64,
vector path, no dot or trace export): O leaves through free tile buffers, 32
features of every wave row at a time, in whole cache lines.

The same call with a routing trace requested takes the variant that stores O
straight from registers; the two must agree bit for bit. The shape puts a
partly valid wave and a wholly invalid one in the last query block
(M = 968 = 7 x 128 + 72), O rows are strided (d + 32 floats, guard values in
the 32 padding floats of every row and in the rows past M), and sampled rows
are checked against the fp64 TileMix oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import GUARD_TRACE, dev, dev_half, guarded

pytestmark = pytest.mark.gpu

HEADS, M, N, G = 2, 968, 777, 2
PAD_ROWS = 40
SENTINEL = np.float32(777.0)


def _codes(rng):
    qt, kt = (M + 15) // 16, (N + 31) // 32
    groups = (kt + G - 1) // G
    return np.repeat(rng.integers(0, 2, (qt, groups)).astype(np.uint8), G, axis=1)[:, :kt].copy()


def _launch(tm, Q, K, V, route, D, precise, with_trace):
    import torch

    ROW = D + 32
    O = torch.full((HEADS, M + PAD_ROWS, ROW), float(SENTINEL), dtype=torch.float32, device="cuda:0")
    K8 = torch.empty((HEADS, N, D), dtype=torch.int8, device="cuda:0")
    ks = torch.empty((HEADS, (N + 63) // 64), dtype=torch.int16, device="cuda:0")
    trace = guarded(HEADS * ((M + 15) // 16) * ((N + 31) // 32), np.uint8, GUARD_TRACE) if with_trace else None
    args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O, heads=HEADS, M=M, N=N, d=D, score_scale=D ** -0.5,
                          o_head_stride=(M + PAD_ROWS) * ROW, o_row_stride=ROW, precise=precise, quantize=2,
                          route_words=dev(route), key_tiles_per_group=G, K8=K8, k_scales=ks,
                          decoded_bits=trace.data_ptr() + 1 if with_trace else None)
    tm.check(tm.quantize_tilemix_qk_batched(None, K, None, K8, None, ks, HEADS, N, N, D), "quantize K")
    tm.check(tm.attention_batched(args), "attention_batched")
    torch.cuda.synchronize()
    return O.cpu().numpy(), K8.cpu().numpy(), ks.cpu().numpy()


@pytest.mark.parametrize("D,precise", [(128, False), (128, True), (64, False), (64, True)],
                         ids=["d128-fast", "d128-precise", "d64-fast", "d64-precise"])
def test_staged_output_matches_direct_stores(tm, oracle_lib, cuda, D, precise):
    from tilemix import routing

    rng = np.random.default_rng(968 + D + precise)
    half = lambda rows: oracle_lib.float_to_half(rng.standard_normal((rows, D)).astype(np.float32))
    q = [half(M) for _ in range(HEADS)]
    k = [half(N) for _ in range(HEADS)]
    v = [half(N) for _ in range(HEADS)]
    codes = np.stack([_codes(rng) for _ in range(HEADS)])
    route = np.concatenate([routing.pack_cells(c, G)[0] for c in codes])
    Q, K, V = dev_half(np.stack(q)), dev_half(np.stack(k)), dev_half(np.stack(v))
    print(f"staged O: heads={HEADS} M={M} N={N} d={D} row={D + 32} precise={precise}", flush=True)
    staged, k8, ks = _launch(tm, Q, K, V, route, D, precise, with_trace=False)
    direct, _, _ = _launch(tm, Q, K, V, route, D, precise, with_trace=True)
    assert np.array_equal(staged.view(np.uint32), direct.view(np.uint32)), "staged and direct O differ"
    assert (staged[:, :, D:] == SENTINEL).all(), "row padding of O written"
    assert (staged[:, M:, :] == SENTINEL).all(), "rows past M written"
    for h in range(HEADS):
        q8, qs = oracle_lib.quantize(q[h], 128)
        rows = np.sort(rng.choice(M, 200, replace=False)).astype(np.int32)
        rows[-1] = M - 1
        expected = oracle_lib.tilemix(q[h], k[h], v[h], q8, k8[h], qs, ks[h].view(np.uint16), codes[h],
                                      float(np.float32(D ** -0.5)), False, rows=rows)
        err = np.abs(staged[h, rows, :D].astype(np.float64) - expected)
        if precise:
            assert (err <= 1e-5 + 1e-4 * np.abs(expected)).all(), (h, float(err.max()))
        else:
            assert err.max() <= 2e-3 and err.mean() <= 2e-4, (h, float(err.max()), float(err.mean()))
