"""A seeded sweep of tilemix_attention_batched over the option space, each case
against the fp64 TileMix oracle.

The hand-picked cases of test_batched_gpu.py fix one option set each; here 24
cases drawn once from a fixed seed combine them (and 8 more with rows of up to
3200 keys): 1-3 heads, ragged M and N,
d from 1 to 128, key_tiles_per_group 1-5, causal or not, skip routes or not,
quantize mode 0 (Q8/K8 given), 1 (both quantized here) or 2 (K8 given, Q
quantized in the kernel), fast or precise P.V, O 16-byte aligned or not, and
a positive, zero or negative score scale (the reference allows both,
src/tests/tilemix_test.cu:343-353). Inputs of every head are followed by 64
NaN rows, so a read past a head's last row shows up in O. Q8/K8/scales and the
decoded route codes must be bit-exact; O is held to the reference's
1e-5 + 1e-4|x| rule with precise P.V and to max-abs 2e-3 / mean-abs 2e-4
(the north star's bound for the fast path, which rounds P to fp16) without.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import GUARD_F32, GUARD_TRACE, compare, dev, dev_half, guarded, guarded_lead, host

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-3, 2e-4
PAD = 64


def _draw(rng, d, max_m, max_n):
    return dict(
        heads=int(rng.integers(1, 4)), M=int(rng.integers(1, max_m)), N=int(rng.integers(1, max_n)),
        d=d, g=int(rng.choice([1, 2, 3, 5])), causal=bool(rng.random() < 0.5),
        p_skip=float(rng.choice([0.0, 0.25])), quantize=int(rng.integers(0, 3)),
        precise=bool(rng.random() < 0.5), aligned=bool(rng.random() < 0.5),
        scale_kind=str(rng.choice(["pos", "pos", "pos", "zero", "neg"])))


def _cases():
    rng = np.random.default_rng(20261202)
    dims = [1, 7, 16, 24, 40, 64, 72, 96, 100, 120, 128]
    # every head dimension at least twice, the other options drawn
    cases = [_draw(rng, dims[i % len(dims)], 700, 900) for i in range(24)]
    # Long rows (up to 50 key tiles): the kernel alternates two V buffers per
    # visited tile and steps over skipped tiles, over many tiles per workgroup.
    long_rng = np.random.default_rng(20261203)
    cases += [_draw(long_rng, [64, 96, 128, 128][i % 4], 3000, 3200) for i in range(8)]
    return cases


CASES = _cases()


def _id(c):
    return (f"h{c['heads']}-{c['M']}x{c['N']}x{c['d']}-g{c['g']}{'-causal' if c['causal'] else ''}"
            f"-skip{c['p_skip']}-q{c['quantize']}{'-precise' if c['precise'] else ''}"
            f"{'-aligned' if c['aligned'] else ''}-{c['scale_kind']}")


def _route_codes(rng, M, N, g, p_skip):
    qt, kt = (M + 15) // 16, (N + 31) // 32
    groups = (kt + g - 1) // g
    u = rng.random((qt, groups))
    codes = np.where(u < p_skip, 2, np.where(u < p_skip + 0.5, 1, 0)).astype(np.uint8)
    return np.repeat(codes, g, axis=1)[:, :kt].copy()


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_batched_sweep_vs_oracle(tm, oracle_lib, cuda, case):
    import torch

    from tilemix import routing

    heads, M, N, d, g = case["heads"], case["M"], case["N"], case["d"], case["g"]
    causal, p_skip, quantize, precise, aligned = (case["causal"], case["p_skip"], case["quantize"],
                                                  case["precise"], case["aligned"])
    rng = np.random.default_rng(M * 1009 + N * 31 + d)
    half = oracle_lib.float_to_half
    q = [half(rng.standard_normal((M, d)).astype(np.float32)) for _ in range(heads)]
    k = [half(rng.standard_normal((N, d)).astype(np.float32)) for _ in range(heads)]
    v = [half(rng.standard_normal((N, d)).astype(np.float32)) for _ in range(heads)]

    def padded(parts, rows):
        out = np.full((heads, rows + PAD, d), 0x7E00, dtype=np.uint16)  # NaN rows between heads
        for h, part in enumerate(parts):
            out[h, :rows] = part
        return out

    Qp, Kp, Vp = padded(q, M), padded(k, N), padded(v, N)
    codes = np.stack([_route_codes(rng, M, N, g, p_skip) for _ in range(heads)])
    packed = [routing.pack_cells(c, g) for c in codes]
    route = np.concatenate([r for r, _ in packed])
    skip = (np.concatenate([s if s is not None else np.zeros(routing.word_count(M, N, g), np.uint64)
                            for _, s in packed]) if p_skip else None)
    base = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    scale = {"pos": base, "zero": 0.0, "neg": -base}[case["scale_kind"]]

    Q, K, V = dev_half(Qp), dev_half(Kp), dev_half(Vp)
    q_stride, k_stride = (M + PAD) * d, (N + PAD) * d
    Q8 = torch.empty((heads, M, d), dtype=torch.int8, device="cuda:0")
    K8 = torch.empty((heads, N, d), dtype=torch.int8, device="cuda:0")
    qs = torch.empty((heads, (M + 127) // 128), dtype=torch.int16, device="cuda:0")
    ks = torch.empty((heads, (N + 63) // 64), dtype=torch.int16, device="cuda:0")
    if quantize == 0:
        tm.check(tm.quantize_tilemix_qk_batched(Q, K, Q8, K8, qs, ks, heads, M, N, d,
                                                q_head_stride=q_stride, k_head_stride=k_stride))
    elif quantize == 2:
        tm.check(tm.quantize_tilemix_qk_batched(None, K, None, K8, None, ks, heads, M, N, d,
                                                k_head_stride=k_stride))
    lead = 4 if aligned else 1
    O = guarded_lead(heads * q_stride, np.float32, GUARD_F32, fill=np.float32(777.0), lead=lead)
    trace = guarded(codes.size, np.uint8, GUARD_TRACE)
    args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O.data_ptr() + 4 * lead, heads=heads, M=M, N=N, d=d,
                          score_scale=scale, q_head_stride=q_stride, k_head_stride=k_stride,
                          v_head_stride=k_stride, o_head_stride=q_stride, causal=causal, precise=precise,
                          quantize=quantize, route_words=dev(route),
                          skip_words=dev(skip) if skip is not None else None, key_tiles_per_group=g,
                          decoded_bits=trace.data_ptr() + 1, Q8=Q8, K8=K8, q_scales=qs, k_scales=ks)
    print(f"sweep {_id(case)}", flush=True)
    tm.check(tm.attention_batched(args))
    torch.cuda.synchronize()

    out = host(O)
    assert (out[:lead] == GUARD_F32).all() and out[-1] == GUARD_F32, "output guard overwritten"
    out = out[lead:-1].reshape(heads, M + PAD, d)
    assert (out[:, M:] == np.float32(777.0)).all(), "head padding of O written"
    got_trace = host(trace)
    assert got_trace[0] == GUARD_TRACE and got_trace[-1] == GUARD_TRACE, "trace guard overwritten"
    assert np.array_equal(got_trace[1:-1].reshape(codes.shape), codes), "decoded route codes differ"
    for h in range(heads):
        q8_ref, qs_ref = oracle_lib.quantize(q[h], 128)
        k8_ref, ks_ref = oracle_lib.quantize(k[h], 64)
        assert np.array_equal(Q8[h].cpu().numpy(), q8_ref), f"head {h}: Q8 differs"
        assert np.array_equal(K8[h].cpu().numpy(), k8_ref), f"head {h}: K8 differs"
        assert np.array_equal(qs[h].cpu().numpy().view(np.uint16), qs_ref), f"head {h}: q_scales differ"
        assert np.array_equal(ks[h].cpu().numpy().view(np.uint16), ks_ref), f"head {h}: k_scales differ"
        expected = oracle_lib.tilemix(q[h], k[h], v[h], q8_ref, k8_ref, qs_ref, ks_ref, codes[h], scale, causal)
        got = out[h, :M]
        assert np.isfinite(got).all(), f"head {h}: non-finite output"
        if precise:
            compare(got, expected, 1e-5, 1e-4, f"head {h} precise vs fp64 oracle")
        else:
            err = np.abs(got.astype(np.float64) - expected)
            assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (h, float(err.max()), float(err.mean()))
    for dev_tensor, original in ((Q, Qp), (K, Kp), (V, Vp)):
        assert np.array_equal(host(dev_tensor), original), "an input was modified"
