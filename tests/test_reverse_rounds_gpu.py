"""Workgroups that walk their key tiles last to first (the batched entry point
on non-causal heads whose query blocks outnumber one XCD's workgroup slots:
every other round of slots on an XCD walks backwards, so it starts on the tiles
the round before it left in that XCD's L2).

The shape puts one query block of each head in a reversed round: 8 heads (one
per XCD), 65 query blocks (the slots of an XCD hold 64), the last one ragged.
Keys end in a partial tile, which the reversed walk visits first; routes are
mixed per cell (g = 1) with skipped groups, so the walk steps over skipped
tiles backwards. Checked against the C oracle: the decoded route codes of
every cell, the INT32 dots of every INT8 cell, and O of the reversed block and
of a sample of forward blocks - fast P.V within 2e-3 / 2e-4, precise P.V within
the reference's 1e-5 + 1e-4|x|.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import GUARD_DOT, GUARD_F32, GUARD_TRACE, dev, dev_half, guarded, guarded_lead, host

pytestmark = pytest.mark.gpu

HEADS, N, D, G = 8, 1000, 128, 1


def _xcd_slots():
    import torch

    return torch.cuda.get_device_properties(0).multi_processor_count // 8 * 2


def _random_codes(rng, M, N, g, p_skip=0.3, p_int8=0.4):
    qt, kt = (M + 15) // 16, (N + 31) // 32
    groups = (kt + g - 1) // g
    u = rng.random((qt, groups))
    group_codes = np.where(u < p_skip, 2, np.where(u < p_skip + p_int8, 1, 0)).astype(np.uint8)
    return np.repeat(group_codes, g, axis=1)[:, :kt].copy()


@pytest.mark.parametrize("precise,lead", [(False, 4), (False, 1), (True, 4)],
                         ids=["fast-vector", "fast-elementwise", "precise-vector"])
def test_reversed_rounds_vs_oracle(tm, oracle_lib, cuda, precise, lead):
    import torch

    from tilemix import routing

    slots = _xcd_slots()
    M = (slots + 1) * 128 - 37  # query block `slots` of every head runs in the second round
    rng = np.random.default_rng(20261202 + lead)
    half = lambda rows: oracle_lib.float_to_half(rng.standard_normal((rows, D)).astype(np.float32))
    q = [half(M) for _ in range(HEADS)]
    k = [half(N) for _ in range(HEADS)]
    v = [half(N) for _ in range(HEADS)]
    codes = np.stack([_random_codes(rng, M, N, G) for _ in range(HEADS)])
    packed = [routing.pack_cells(c, G) for c in codes]
    route = np.concatenate([p[0] for p in packed])
    skip = np.concatenate([p[1] if p[1] is not None else np.zeros(routing.word_count(M, N, G), np.uint64)
                           for p in packed])
    Q, K, V = dev_half(np.stack(q)), dev_half(np.stack(k)), dev_half(np.stack(v))
    O = guarded_lead(HEADS * M * D, np.float32, GUARD_F32, fill=np.nan, lead=lead)
    Q8 = torch.empty((HEADS, M, D), dtype=torch.int8, device="cuda:0")
    K8 = torch.empty((HEADS, N, D), dtype=torch.int8, device="cuda:0")
    qs = torch.empty((HEADS, (M + 127) // 128), dtype=torch.int16, device="cuda:0")
    ks = torch.empty((HEADS, (N + 63) // 64), dtype=torch.int16, device="cuda:0")
    trace = guarded(codes.size, np.uint8, GUARD_TRACE)
    dots = guarded(HEADS * M * N, np.int32, GUARD_DOT)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O.data_ptr() + 4 * lead, heads=HEADS, M=M, N=N, d=D,
                          score_scale=scale, causal=False, precise=precise, quantize=1, route_words=dev(route),
                          skip_words=dev(skip), key_tiles_per_group=G, decoded_bits=trace.data_ptr() + 1,
                          score_dots=dots.data_ptr() + 4, Q8=Q8, K8=K8, q_scales=qs, k_scales=ks)
    print(f"reversed rounds: heads={HEADS} M={M} N={N} d={D} slots={slots} precise={precise} lead={lead}",
          flush=True)
    tm.check(tm.attention_batched(args), "attention_batched")
    torch.cuda.synchronize()

    got_trace = host(trace)
    assert got_trace[0] == GUARD_TRACE and got_trace[-1] == GUARD_TRACE
    assert np.array_equal(got_trace[1:-1].reshape(codes.shape), codes), "decoded route codes"
    out = host(O)
    assert (out[:lead] == GUARD_F32).all() and out[-1] == GUARD_F32, "output guard overwritten"
    out = out[lead:-1].reshape(HEADS, M, D)
    all_dots = host(dots)
    assert all_dots[0] == GUARD_DOT and all_dots[-1] == GUARD_DOT
    all_dots = all_dots[1:-1].reshape(HEADS, M, N)
    reversed_rows = np.arange(slots * 128, M)
    for h in range(HEADS):
        q8_ref, qs_ref = oracle_lib.quantize(q[h], 128)
        k8_ref, ks_ref = oracle_lib.quantize(k[h], 64)
        assert np.array_equal(Q8[h].cpu().numpy(), q8_ref) and np.array_equal(K8[h].cpu().numpy(), k8_ref)
        cells = np.repeat(np.repeat(codes[h] == 1, 16, axis=0)[:M], 32, axis=1)[:, :N]
        # |dot| <= 127^2 * 128 < 2^53: exact in float64
        exact = (q8_ref.astype(np.float64) @ k8_ref.astype(np.float64).T).astype(np.int64)
        want = np.where(cells, exact, int(GUARD_DOT)).astype(np.int32)
        assert np.array_equal(all_dots[h], want), f"head {h}: INT32 dots"
        forward_rows = np.sort(rng.choice(slots * 128, 256, replace=False))
        rows = np.concatenate([forward_rows, reversed_rows]).astype(np.int32)
        expected = oracle_lib.tilemix(q[h], k[h], v[h], q8_ref, k8_ref, qs_ref, ks_ref, codes[h], scale, False,
                                      rows=rows)
        got = out[h, rows].astype(np.float64)
        assert np.isfinite(got).all(), f"head {h}: non-finite output"
        err = np.abs(got - expected)
        if precise:
            bad = err > 1e-5 + 1e-4 * np.abs(expected)
            assert not bad.any(), f"head {h}: {int(bad.sum())} elements outside 1e-5 + 1e-4|x|"
        else:
            assert err.max() <= 2e-3 and err.mean() <= 2e-4, (h, float(err.max()), float(err.mean()))
