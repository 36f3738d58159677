"""GPU parity of the batched entry point (tilemix_attention_batched) and the
BASELINE workloads, through the C ABI, against the C oracle:

* configs 1 and 2 in full and configs 3-5 on a seeded sample of >= 4096
  (head, row) pairs: Q8/K8/q_scales/k_scales bit-exact for every head, outputs
  within max-abs 2e-3 / mean-abs 2e-4 of the fp64 TileMix oracle (fast P.V);
* int32 score dots of two config-2 heads in full, bit-exact;
* the batched call equals the per-head reference API head by head (same
  inputs, same flags: identical bits);
* the skip / causal extensions against the oracle's definitions, including
  rows left without a visible key, ragged sizes and the decoded route codes;
* head strides with padding, guards around every output, inputs unchanged;
* quantize modes 0 / 1 / 2 agree, and the precise P.V mode meets the
  reference's 1e-5 + 1e-4|x| rule.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from helpers import GUARD_DOT, GUARD_F32, GUARD_TRACE, compare, dev, dev_half, guarded, guarded_lead, host

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-3, 2e-4


def f16_bits(t) -> np.ndarray:
    import torch

    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def run_workload(tm, w, seed, precise=False):
    import torch

    from tilemix import workloads

    Q, K, V = workloads.make_inputs(w, seed)
    codes = workloads.make_codes(w, seed, Q, K)
    route_np, skip_np = workloads.pack_heads(codes, w.key_tiles_per_group)
    heads, S, D = w.heads, w.S, w.D
    dev_ = "cuda:0"
    O = torch.empty((heads, S, D), dtype=torch.float32, device=dev_)
    Q8 = torch.empty((heads, S, D), dtype=torch.int8, device=dev_)
    K8 = torch.empty((heads, S, D), dtype=torch.int8, device=dev_)
    qs = torch.empty((heads, (S + 127) // 128), dtype=torch.int16, device=dev_)
    ks = torch.empty((heads, (S + 63) // 64), dtype=torch.int16, device=dev_)
    args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O, heads=heads, M=S, N=S, d=D, score_scale=w.score_scale,
                          causal=w.causal, precise=precise, quantize=1, route_words=dev(route_np),
                          skip_words=dev(skip_np) if skip_np is not None else None,
                          key_tiles_per_group=w.key_tiles_per_group, Q8=Q8, K8=K8, q_scales=qs, k_scales=ks)
    print(f"workload {w.describe()} seed={seed} precise={precise}", flush=True)
    tm.check(tm.attention_batched(args), "attention_batched")
    torch.cuda.synchronize()
    return dict(q=f16_bits(Q), k=f16_bits(K), v=f16_bits(V), o=O.cpu().numpy(), q8=Q8.cpu().numpy(),
                k8=K8.cpu().numpy(), qs=f16_bits(qs), ks=f16_bits(ks), codes=codes)


def check_workload(oracle_lib, w, r, sample_rows=None, seed=0):
    heads, S = w.heads, w.S
    for h in range(heads):
        q8_ref, qs_ref = oracle_lib.quantize(r["q"][h], 128)
        k8_ref, ks_ref = oracle_lib.quantize(r["k"][h], 64)
        assert np.array_equal(r["q8"][h], q8_ref), f"Q8 head {h}"
        assert np.array_equal(r["k8"][h], k8_ref), f"K8 head {h}"
        assert np.array_equal(r["qs"][h], qs_ref) and np.array_equal(r["ks"][h], ks_ref), f"scales head {h}"
    rng = np.random.default_rng(seed)
    if sample_rows is None:
        plan = [(h, None) for h in range(heads)]
    else:
        chosen = sorted(set(rng.choice(heads, size=min(heads, 8), replace=False).tolist()))
        per = -(-sample_rows // len(chosen))
        plan = [(h, np.sort(rng.choice(S, size=per, replace=False)).astype(np.int32)) for h in chosen]
    max_abs, total, count = 0.0, 0.0, 0
    for h, rows in plan:
        expected = oracle_lib.tilemix(r["q"][h], r["k"][h], r["v"][h], r["q8"][h], r["k8"][h], r["qs"][h],
                                      r["ks"][h], r["codes"][h], w.score_scale, w.causal, rows=rows)
        got = r["o"][h] if rows is None else r["o"][h][rows]
        assert np.isfinite(got).all()
        err = np.abs(got.astype(np.float64) - expected)
        max_abs = max(max_abs, float(err.max()))
        total += float(err.sum())
        count += err.size
    mean_abs = total / count
    print(f"{w.describe()}: rows checked {count // w.D}, max_abs {max_abs:.3g}, mean_abs {mean_abs:.3g}")
    assert max_abs <= MAX_ABS and mean_abs <= MEAN_ABS, (max_abs, mean_abs)
    if sample_rows is not None:
        assert count // w.D >= sample_rows


@pytest.mark.parametrize("config", [1, 2])
def test_workload_full(tm, oracle_lib, cuda, config):
    from tilemix import workloads

    w = workloads.WORKLOADS[config]
    check_workload(oracle_lib, w, run_workload(tm, w, seed=100 + config))


@pytest.mark.parametrize("config", [3, 4, 5])
def test_workload_sampled(tm, oracle_lib, cuda, config):
    from tilemix import workloads

    w = workloads.WORKLOADS[config]
    check_workload(oracle_lib, w, run_workload(tm, w, seed=100 + config), sample_rows=4096, seed=config)


def test_workload_precise_meets_reference_rule(tm, oracle_lib, cuda):
    from tilemix import workloads

    w = workloads.WORKLOADS[1]
    r = run_workload(tm, w, seed=11, precise=True)
    for h in range(w.heads):
        expected = oracle_lib.tilemix(r["q"][h], r["k"][h], r["v"][h], r["q8"][h], r["k8"][h], r["qs"][h],
                                      r["ks"][h], r["codes"][h], w.score_scale)
        compare(r["o"][h], expected, 1e-5, 1e-4, f"precise head {h}")


def test_score_dots_two_heads_full(tm, oracle_lib, cuda):
    """Config 2 shape (S=2048, D=64), two heads, every int32 dot of every INT8 cell."""
    import torch

    from tilemix import routing, workloads

    w = workloads.WORKLOADS[2]
    heads, S, D = 2, w.S, w.D
    rng = np.random.default_rng(5)
    q = [oracle_lib.float_to_half(rng.standard_normal((S, D)).astype(np.float32)) for _ in range(heads)]
    k = [oracle_lib.float_to_half(rng.standard_normal((S, D)).astype(np.float32)) for _ in range(heads)]
    v = [oracle_lib.float_to_half(rng.standard_normal((S, D)).astype(np.float32)) for _ in range(heads)]
    codes = np.stack([routing.bernoulli_tiles(rng, S, S, 64, 64) for _ in range(heads)])
    route_np, _ = workloads.pack_heads(codes, 2)
    Q, K, V = (dev_half(np.stack(x)) for x in (q, k, v))
    O = torch.empty((heads, S, D), dtype=torch.float32, device="cuda:0")
    Q8 = torch.empty((heads, S, D), dtype=torch.int8, device="cuda:0")
    K8 = torch.empty((heads, S, D), dtype=torch.int8, device="cuda:0")
    qs = torch.empty((heads, S // 128), dtype=torch.int16, device="cuda:0")
    ks = torch.empty((heads, S // 64), dtype=torch.int16, device="cuda:0")
    tm.check(tm.quantize_tilemix_qk_batched(Q, K, Q8, K8, qs, ks, heads, S, S, D))
    dots = guarded(heads * S * S, np.int32, GUARD_DOT)
    args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O, heads=heads, M=S, N=S, d=D, score_scale=w.score_scale, quantize=0,
                          route_words=dev(route_np), key_tiles_per_group=2, Q8=Q8, K8=K8, q_scales=qs,
                          k_scales=ks, score_dots=dots.data_ptr() + 4)
    print("score dots: 2 heads S=2048 D=64", flush=True)
    tm.check(tm.attention_batched(args))
    torch.cuda.synchronize()
    got = host(dots)
    assert got[0] == GUARD_DOT and got[-1] == GUARD_DOT
    got = got[1:-1].reshape(heads, S, S)
    for h in range(heads):
        q8_ref, _ = oracle_lib.quantize(q[h], 128)
        k8_ref, _ = oracle_lib.quantize(k[h], 64)
        assert np.array_equal(Q8[h].cpu().numpy(), q8_ref) and np.array_equal(K8[h].cpu().numpy(), k8_ref)
        cell = np.repeat(np.repeat(codes[h] == routing.INT8, 16, axis=0), 32, axis=1)
        exact = (q8_ref.astype(np.int64) @ k8_ref.astype(np.int64).T).astype(np.int32)
        expected = np.where(cell, exact, np.int32(GUARD_DOT))
        bad = got[h] != expected
        assert not bad.any(), f"head {h}: {int(bad.sum())} dots differ, first {np.argwhere(bad)[:3].tolist()}"


def random_codes(rng, M, N, g, p_skip=0.0, p_int8=0.5):
    qt, kt = (M + 15) // 16, (N + 31) // 32
    groups = (kt + g - 1) // g
    u = rng.random((qt, groups))
    group_codes = np.where(u < p_skip, 2, np.where(u < p_skip + p_int8, 1, 0)).astype(np.uint8)
    return np.repeat(group_codes, g, axis=1)[:, :kt].copy()


def make_problem(oracle_lib, heads, M, N, d, seed, pad=0):
    """Per-head fp16 inputs and head strides with `pad` spare rows between heads."""
    rng = np.random.default_rng(seed)
    q = [oracle_lib.float_to_half(rng.standard_normal((M, d)).astype(np.float32)) for _ in range(heads)]
    k = [oracle_lib.float_to_half(rng.standard_normal((N, d)).astype(np.float32)) for _ in range(heads)]
    v = [oracle_lib.float_to_half(rng.standard_normal((N, d)).astype(np.float32)) for _ in range(heads)]

    def padded(parts, rows):
        out = np.full((heads, rows + pad, d), 0x7E00, dtype=np.uint16)  # NaN padding: must never be read
        for h, p in enumerate(parts):
            out[h, :rows] = p
        return out

    return q, k, v, padded(q, M), padded(k, N), padded(v, N), rng


BATCH_CASES = [
    # heads, M, N, d, g, causal, p_skip
    (3, 300, 300, 64, 2, True, 0.0),
    (2, 1000, 1000, 128, 2, True, 0.2),
    (4, 77, 333, 128, 1, False, 0.3),
    (2, 129, 4099, 64, 3, False, 0.0),
    (3, 260, 260, 96, 1, True, 0.4),
    (1, 4096, 4096, 128, 2, True, 0.0),
    (2, 77, 333, 128, 1, True, 0.3),   # causal with fewer queries than keys
    (2, 500, 130, 64, 2, True, 0.0),   # causal with more queries than keys
    (2, 200, 333, 112, 2, True, 0.2),  # d > 96 with the last 16-byte chunks of each row absent
    (2, 150, 270, 100, 1, False, 0.0), # d > 96 on the element-wise path (d % 16 != 0)
]


# Each case runs with O at a 4-byte offset (element-wise path) and 16-byte
# aligned (the vector path when d % 16 == 0); the 64 NaN rows between heads
# cover every row a head's last 64-key tile could reach past N.
BATCH_RUNS = [c + (aligned,) for c in BATCH_CASES for aligned in (False, True)]


@pytest.mark.parametrize("heads,M,N,d,g,causal,p_skip,aligned", BATCH_RUNS,
                         ids=[f"h{c[0]}-{c[1]}x{c[2]}x{c[3]}-g{c[4]}{'-causal' if c[5] else ''}-skip{c[6]}"
                              f"{'-aligned' if c[7] else ''}" for c in BATCH_RUNS])
def test_batched_extensions_vs_oracle(tm, oracle_lib, cuda, heads, M, N, d, g, causal, p_skip, aligned):
    """Skip words, causal masking, ragged sizes, padded head strides, fused
    quantization (mode 1) with Q8/q_scales outputs, decoded route codes."""
    import torch

    from tilemix import routing

    pad = 64
    lead = 4 if aligned else 1
    q, k, v, Qp, Kp, Vp, rng = make_problem(oracle_lib, heads, M, N, d, seed=M * N + d, pad=pad)
    codes = np.stack([random_codes(rng, M, N, g, p_skip) for _ in range(heads)])
    if p_skip:
        codes[0, 0, :] = routing.SKIP  # the first 16 rows of head 0 see no key at all
    route = np.concatenate([routing.pack_cells(c, g)[0] for c in codes])
    skip_parts = [routing.pack_cells(c, g)[1] for c in codes]
    skip = (np.concatenate([s if s is not None else np.zeros(routing.word_count(M, N, g), np.uint64)
                            for s in skip_parts]) if p_skip else None)
    Q, K, V = dev_half(Qp), dev_half(Kp), dev_half(Vp)
    o_stride = (M + pad) * d
    O = guarded_lead(heads * o_stride, np.float32, GUARD_F32, fill=np.float32(777.0), lead=lead)
    Q8 = torch.empty((heads, M, d), dtype=torch.int8, device="cuda:0")
    K8 = torch.empty((heads, N, d), dtype=torch.int8, device="cuda:0")
    qs = torch.empty((heads, (M + 127) // 128), dtype=torch.int16, device="cuda:0")
    ks = torch.empty((heads, (N + 63) // 64), dtype=torch.int16, device="cuda:0")
    cells = codes[0].size
    trace = guarded(heads * cells, np.uint8, GUARD_TRACE)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O.data_ptr() + 4 * lead, heads=heads, M=M, N=N, d=d,
                          score_scale=scale,
                          q_head_stride=(M + pad) * d, k_head_stride=(N + pad) * d, v_head_stride=(N + pad) * d,
                          o_head_stride=o_stride, causal=causal, quantize=1, route_words=dev(route),
                          skip_words=dev(skip) if skip is not None else None, key_tiles_per_group=g,
                          decoded_bits=trace.data_ptr() + 1, Q8=Q8, K8=K8, q_scales=qs, k_scales=ks)
    print(f"batched heads={heads} M={M} N={N} d={d} g={g} causal={causal} p_skip={p_skip} aligned={aligned}",
          flush=True)
    tm.check(tm.attention_batched(args))
    torch.cuda.synchronize()
    out = host(O)
    assert (out[:lead] == GUARD_F32).all() and out[-1] == GUARD_F32, "output guard overwritten"
    out = out[lead:-1].reshape(heads, M + pad, d)
    assert (out[:, M:] == np.float32(777.0)).all(), "head padding of O written"
    got_trace = host(trace)
    assert got_trace[0] == GUARD_TRACE and got_trace[-1] == GUARD_TRACE
    assert np.array_equal(got_trace[1:-1].reshape(codes.shape), codes), "decoded route codes differ"
    for h in range(heads):
        q8_ref, qs_ref = oracle_lib.quantize(q[h], 128)
        k8_ref, ks_ref = oracle_lib.quantize(k[h], 64)
        assert np.array_equal(Q8[h].cpu().numpy(), q8_ref) and np.array_equal(K8[h].cpu().numpy(), k8_ref)
        assert np.array_equal(f16_bits(qs[h]), qs_ref) and np.array_equal(f16_bits(ks[h]), ks_ref)
        rows = None if M <= 1200 else np.sort(rng.choice(M, 1024, replace=False)).astype(np.int32)
        expected = oracle_lib.tilemix(q[h], k[h], v[h], q8_ref, k8_ref, qs_ref, ks_ref, codes[h], scale, causal,
                                      rows=rows)
        got = out[h, :M] if rows is None else out[h, rows]
        assert np.isfinite(got).all()
        err = np.abs(got.astype(np.float64) - expected)
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (h, float(err.max()), float(err.mean()))
    if p_skip:
        assert not out[0, :16].any(), "rows without a visible key must be zero"
    for dev_tensor, original in ((Q, Qp), (K, Kp), (V, Vp)):
        assert np.array_equal(host(dev_tensor), original), "an input was modified"


def test_batched_equals_per_head_api(tm, oracle_lib, cuda):
    """Each head of one batched launch is bit-identical to the reference API on that head."""
    import torch

    from tilemix import routing

    heads, M, N, d, g = 3, 200, 333, 96, 2
    q, k, v, Qp, Kp, Vp, rng = make_problem(oracle_lib, heads, M, N, d, seed=9)
    codes = np.stack([random_codes(rng, M, N, g) for _ in range(heads)])
    route = [routing.pack_cells(c, g)[0] for c in codes]
    Q, K, V = dev_half(Qp), dev_half(Kp), dev_half(Vp)
    Q8 = torch.empty((heads, M, d), dtype=torch.int8, device="cuda:0")
    K8 = torch.empty((heads, N, d), dtype=torch.int8, device="cuda:0")
    qs = torch.empty((heads, 2), dtype=torch.int16, device="cuda:0")
    ks = torch.empty((heads, 6), dtype=torch.int16, device="cuda:0")
    tm.check(tm.quantize_tilemix_qk_batched(Q, K, Q8, K8, qs, ks, heads, M, N, d))
    scale = 0.125
    O = torch.empty((heads, M, d), dtype=torch.float32, device="cuda:0")
    # FP16 cells leave their dots untouched, so both sides start from the guard value.
    dots = torch.full((heads, M, N), int(GUARD_DOT), dtype=torch.int32, device="cuda:0")
    trace = torch.full((heads, codes[0].size), int(GUARD_TRACE), dtype=torch.uint8, device="cuda:0")
    args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O, heads=heads, M=M, N=N, d=d, score_scale=scale, precise=True,
                          quantize=0, route_words=dev(np.concatenate(route)), key_tiles_per_group=g,
                          decoded_bits=trace, Q8=Q8, K8=K8, q_scales=qs, k_scales=ks, score_dots=dots)
    print("batched vs per-head", flush=True)
    tm.check(tm.attention_batched(args))
    for h in range(heads):
        O1 = torch.empty((M, d), dtype=torch.float32, device="cuda:0")
        dots1 = torch.full((M, N), int(GUARD_DOT), dtype=torch.int32, device="cuda:0")
        trace1 = torch.full((codes[0].size,), int(GUARD_TRACE), dtype=torch.uint8, device="cuda:0")
        words = dev(route[h])
        tm.check(tm.launch_fused_fp16_attention(
            Q[h], K[h], V[h], O1, M, N, d, scale,
            routing=tm.TileMixRouting(words, route[h].size, g, trace1),
            quantized=tm.TileMixQuantized(Q8[h], K8[h], qs[h], ks[h], dots1)))
        torch.cuda.synchronize()
        assert np.array_equal(O[h].cpu().numpy().view(np.uint32), O1.cpu().numpy().view(np.uint32)), f"O head {h}"
        assert torch.equal(dots[h], dots1) and torch.equal(trace[h], trace1), f"dots/trace head {h}"


def test_quantize_modes_agree(tm, oracle_lib, cuda):
    """Mode 1 (quantize Q and K), 2 (K8 given) and 0 (all given) give identical bits."""
    import torch

    from tilemix import routing

    heads, M, N, d, g = 2, 384, 500, 128, 2
    q, k, v, Qp, Kp, Vp, rng = make_problem(oracle_lib, heads, M, N, d, seed=21)
    codes = np.stack([random_codes(rng, M, N, g, p_skip=0.1) for _ in range(heads)])
    packed = [routing.pack_cells(c, g) for c in codes]
    route = dev(np.concatenate([r for r, _ in packed]))
    skip = dev(np.concatenate([s for _, s in packed]))
    Q, K, V = dev_half(Qp), dev_half(Kp), dev_half(Vp)
    outs = []
    Q8 = torch.empty((heads, M, d), dtype=torch.int8, device="cuda:0")
    K8 = torch.empty((heads, N, d), dtype=torch.int8, device="cuda:0")
    qs = torch.empty((heads, 3), dtype=torch.int16, device="cuda:0")
    ks = torch.empty((heads, 8), dtype=torch.int16, device="cuda:0")
    for mode in (1, 2, 0):
        O = torch.empty((heads, M, d), dtype=torch.float32, device="cuda:0")
        if mode == 0:
            tm.check(tm.quantize_tilemix_qk_batched(Q, K, Q8, K8, qs, ks, heads, M, N, d))
        kw = dict(Q8=Q8 if mode != 2 else None, q_scales=qs if mode != 2 else None, K8=K8, k_scales=ks)
        args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O, heads=heads, M=M, N=N, d=d, score_scale=0.09, quantize=mode,
                              route_words=route, skip_words=skip, key_tiles_per_group=g, **kw)
        print(f"quantize mode {mode}", flush=True)
        tm.check(tm.attention_batched(args))
        torch.cuda.synchronize()
        outs.append(O.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.array_equal(outs[0].view(np.uint32), outs[2].view(np.uint32))
    for h in range(heads):
        q8_ref, qs_ref = oracle_lib.quantize(q[h], 128)
        k8_ref, ks_ref = oracle_lib.quantize(k[h], 64)
        expected = oracle_lib.tilemix(q[h], k[h], v[h], q8_ref, k8_ref, qs_ref, ks_ref, codes[h], 0.09)
        err = np.abs(outs[0][h].astype(np.float64) - expected)
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS


def test_batched_without_routes_is_dense(tm, oracle_lib, cuda):
    """No route words: every cell FP16, no quantized operands needed (causal and not)."""
    import torch

    heads, M, N, d = 2, 150, 150, 40
    q, k, v, Qp, Kp, Vp, _ = make_problem(oracle_lib, heads, M, N, d, seed=33)
    Q, K, V = dev_half(Qp), dev_half(Kp), dev_half(Vp)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    for causal in (False, True):
        O = torch.empty((heads, M, d), dtype=torch.float32, device="cuda:0")
        args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O, heads=heads, M=M, N=N, d=d, score_scale=scale,
                              causal=causal, precise=True, quantize=0)
        print(f"dense batched causal={causal}", flush=True)
        tm.check(tm.attention_batched(args))
        torch.cuda.synchronize()
        for h in range(heads):
            expected = oracle_lib.tilemix(q[h], k[h], v[h], score_scale=scale, causal=causal)
            compare(O[h].cpu().numpy(), expected, 1e-5, 1e-4, f"dense causal={causal} head {h}")
