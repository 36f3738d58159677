"""GPU checks of the batched entry point's layout and output options:

* fp16 / bf16 O equal the fp32 O rounded to nearest even, bit for bit;
* row-strided [S, H, D] tensors (head stride D, row stride H * D) give the
  same O, Q8/K8 and scales as the contiguous [H, S, D] layout, bit for bit,
  on the vector (d % 16 == 0) and element-wise (odd d) paths;
* tilemix_quantize_qk_strided equals the contiguous batched quantizer;
* a head whose K / V span more than 2 GiB (4 MiB row stride) takes the
  element-wise path and gives the contiguous run's bits;
* a seeded sweep of 12 more shapes (ragged S, d from 8 to 128, causal,
  precise, routed, fp16 or bf16 O) holds both of the first two properties.
"""
from __future__ import annotations

import numpy as np
import pytest

from tilemix import routing

pytestmark = pytest.mark.gpu


def _inputs(torch, heads, S, d, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return [torch.randn(heads, S, d, generator=g, device="cuda").half() for _ in range(3)]


def _routes(torch, heads, S, g, seed):
    rng = np.random.default_rng(seed)
    words = []
    for _ in range(heads):
        r, _ = routing.pack_cells(routing.bernoulli_tiles(rng, S, S, 64, 64, 0.5), g)
        words.append(r)
    return torch.from_numpy(np.concatenate(words).view(np.int64)).cuda()


def _run(tm, torch, Q, K, V, heads, S, d, dtype, layout, causal=False, precise=False, route=None, g=2):
    """Attention over [H, S, D] inputs, presented in `layout` ("hsd" or "shd")."""
    torch_dtype = {tm.DTYPE_F32: torch.float32, tm.DTYPE_F16: torch.float16, tm.DTYPE_BF16: torch.bfloat16}[dtype]
    K8 = torch.zeros(heads, S, d, dtype=torch.int8, device="cuda")
    ks = torch.zeros(heads, (S + 63) // 64, dtype=torch.int16, device="cuda")
    Q8 = torch.zeros(heads, S, d, dtype=torch.int8, device="cuda")
    qs = torch.zeros(heads, (S + 127) // 128, dtype=torch.int16, device="cuda")
    kw = dict(heads=heads, M=S, N=S, d=d, score_scale=d ** -0.5, causal=causal, precise=precise, quantize=1,
              route_words=route, key_tiles_per_group=g, K8=K8, k_scales=ks, Q8=Q8, q_scales=qs, o_dtype=dtype)
    if layout == "hsd":
        O = torch.full((heads, S, d), float("nan"), device="cuda").to(torch_dtype)
        args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O, **kw)
    else:
        q, k, v = (t.permute(1, 0, 2).contiguous() for t in (Q, K, V))  # [S, H, D]
        O = torch.full((S, heads, d), float("nan"), device="cuda").to(torch_dtype)
        args = tm.BatchedArgs(Q=q, K=k, V=v, O=O, q_head_stride=d, k_head_stride=d, v_head_stride=d,
                              o_head_stride=d, q_row_stride=heads * d, k_row_stride=heads * d,
                              v_row_stride=heads * d, o_row_stride=heads * d, **kw)
    tm.check(tm.attention_batched(args), "attention")
    torch.cuda.synchronize()
    out = O if layout == "hsd" else O.permute(1, 0, 2)
    return out.contiguous().cpu(), Q8.cpu(), qs.cpu(), K8.cpu(), ks.cpu()


@pytest.mark.parametrize("heads,S,d,causal,precise,routed", [
    (4, 512, 64, False, False, True), (2, 1024, 128, True, False, True), (3, 300, 128, False, True, False),
    (2, 257, 48, True, False, True),
])
def test_fp16_bf16_output_equals_rounded_fp32(tm, cuda, heads, S, d, causal, precise, routed):
    import torch

    print(f"output dtypes heads={heads} S={S} d={d} causal={causal} precise={precise} routed={routed}", flush=True)
    Q, K, V = _inputs(torch, heads, S, d, S + d)
    route = _routes(torch, heads, S, 2, 5) if routed else None
    o32 = _run(tm, torch, Q, K, V, heads, S, d, tm.DTYPE_F32, "hsd", causal, precise, route)[0]
    o16 = _run(tm, torch, Q, K, V, heads, S, d, tm.DTYPE_F16, "hsd", causal, precise, route)[0]
    ob16 = _run(tm, torch, Q, K, V, heads, S, d, tm.DTYPE_BF16, "hsd", causal, precise, route)[0]
    assert torch.isfinite(o32).all()
    assert torch.equal(o16.view(torch.int16), o32.half().view(torch.int16))
    assert torch.equal(ob16.view(torch.int16), o32.bfloat16().view(torch.int16))


@pytest.mark.parametrize("heads,S,d,causal,dtype", [
    (4, 512, 64, False, 0), (8, 1024, 128, True, 0), (4, 384, 128, False, 2), (3, 200, 17, True, 0),
    (2, 130, 40, False, 1),
])
def test_row_strided_layout_equals_contiguous(tm, cuda, heads, S, d, causal, dtype):
    import torch

    print(f"[S,H,D] layout heads={heads} S={S} d={d} causal={causal} dtype={dtype}", flush=True)
    Q, K, V = _inputs(torch, heads, S, d, 3 * S + d)
    route = _routes(torch, heads, S, 2, 11)
    a = _run(tm, torch, Q, K, V, heads, S, d, dtype, "hsd", causal, False, route)
    b = _run(tm, torch, Q, K, V, heads, S, d, dtype, "shd", causal, False, route)
    names = ("O", "Q8", "q_scales", "K8", "k_scales")
    for name, x, y in zip(names, a, b):
        if x.dtype.is_floating_point:
            assert torch.equal(x.view(torch.int16 if x.element_size() == 2 else torch.int32),
                               y.view(torch.int16 if y.element_size() == 2 else torch.int32)), name
        else:
            assert torch.equal(x, y), name


@pytest.mark.parametrize("heads,M,N,d", [(4, 256, 512, 128), (3, 100, 70, 24), (2, 128, 64, 17)])
def test_strided_quantizer_equals_contiguous(tm, cuda, heads, M, N, d):
    import torch

    print(f"strided quantizer heads={heads} M={M} N={N} d={d}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(M * N + d)
    Q = torch.randn(heads, M, d, generator=g, device="cuda").half()
    K = torch.randn(heads, N, d, generator=g, device="cuda").half()
    outs = []
    for strided in (False, True):
        q8 = torch.zeros(heads, M, d, dtype=torch.int8, device="cuda")
        k8 = torch.zeros(heads, N, d, dtype=torch.int8, device="cuda")
        qs = torch.zeros(heads, (M + 127) // 128, dtype=torch.int16, device="cuda")
        ks = torch.zeros(heads, (N + 63) // 64, dtype=torch.int16, device="cuda")
        if strided:
            q, k = Q.permute(1, 0, 2).contiguous(), K.permute(1, 0, 2).contiguous()
            rc = tm.quantize_tilemix_qk_strided(q, k, q8, k8, qs, ks, heads, M, N, d, d, d, heads * d, heads * d)
        else:
            rc = tm.quantize_tilemix_qk_batched(Q, K, q8, k8, qs, ks, heads, M, N, d)
        tm.check(rc, "quantize")
        torch.cuda.synchronize()
        outs.append([t.cpu() for t in (q8, k8, qs, ks)])
    for x, y in zip(*outs):
        assert torch.equal(x, y)


def test_heads_past_2gib_take_the_elementwise_path(tm, cuda):
    """K and V rows 4 MiB apart, so a head spans more than 2 GiB: the vector
    path's 32-bit buffer offsets cannot address it, the launch takes the
    element-wise path, and O, Q8/K8 and scales equal the contiguous run's."""
    import torch

    heads, S, d = 1, 1024, 64
    stride = (1 << 21) + 64  # elements between consecutive rows
    print(f"huge row stride S={S} d={d} stride={stride}", flush=True)
    Q, K, V = _inputs(torch, heads, S, d, 99)
    route = _routes(torch, heads, S, 2, 21)
    ref = _run(tm, torch, Q, K, V, heads, S, d, tm.DTYPE_F32, "hsd", False, False, route)
    k_big = torch.empty(S * stride, dtype=torch.float16, device="cuda")
    v_big = torch.empty(S * stride, dtype=torch.float16, device="cuda")
    k_big.as_strided((S, d), (stride, 1)).copy_(K[0])
    v_big.as_strided((S, d), (stride, 1)).copy_(V[0])
    O = torch.full((heads, S, d), float("nan"), device="cuda")
    K8 = torch.zeros(heads, S, d, dtype=torch.int8, device="cuda")
    ks = torch.zeros(heads, (S + 63) // 64, dtype=torch.int16, device="cuda")
    Q8 = torch.zeros(heads, S, d, dtype=torch.int8, device="cuda")
    qs = torch.zeros(heads, (S + 127) // 128, dtype=torch.int16, device="cuda")
    args = tm.BatchedArgs(Q=Q, K=k_big, V=v_big, O=O, heads=heads, M=S, N=S, d=d, score_scale=d ** -0.5,
                          quantize=1, route_words=route, key_tiles_per_group=2, K8=K8, k_scales=ks, Q8=Q8,
                          q_scales=qs, k_row_stride=stride, v_row_stride=stride)
    tm.check(tm.attention_batched(args), "attention")
    torch.cuda.synchronize()
    got = (O.cpu(), Q8.cpu(), qs.cpu(), K8.cpu(), ks.cpu())
    del k_big, v_big
    for name, x, y in zip(("O", "Q8", "q_scales", "K8", "k_scales"), ref, got):
        if x.dtype.is_floating_point:
            assert torch.equal(x.view(torch.int32), y.view(torch.int32)), name
        else:
            assert torch.equal(x, y), name


def _layout_cases():
    rng = np.random.default_rng(20261203)
    dims = [8, 17, 32, 48, 64, 96, 100, 128]
    cases = []
    for i in range(12):  # every head dimension at least once, the other options drawn
        cases.append((int(rng.integers(1, 5)), int(rng.integers(1, 700)), dims[i % len(dims)],
                      bool(rng.random() < 0.5), bool(rng.random() < 0.5), bool(rng.random() < 0.7),
                      int(rng.integers(1, 3))))
    return cases


LAYOUT_CASES = _layout_cases()


@pytest.mark.parametrize("heads,S,d,causal,precise,routed,dtype", LAYOUT_CASES,
                         ids=[f"h{c[0]}-S{c[1]}-d{c[2]}{'-causal' if c[3] else ''}{'-precise' if c[4] else ''}"
                              f"{'-routed' if c[5] else ''}-{'f16' if c[6] == 1 else 'bf16'}" for c in LAYOUT_CASES])
def test_layout_and_output_type_sweep(tm, cuda, heads, S, d, causal, precise, routed, dtype):
    """Seeded shapes: the row-strided [S, H, D] run equals the contiguous [H, S, D] run bit for bit
    (O, Q8/K8 and scales), and its fp16 / bf16 O equals the contiguous fp32 O rounded."""
    import torch

    print(f"layout sweep heads={heads} S={S} d={d} causal={causal} precise={precise} routed={routed} "
          f"dtype={dtype}", flush=True)
    Q, K, V = _inputs(torch, heads, S, d, 7 * S + d)
    route = _routes(torch, heads, S, 2, S) if routed else None
    ref = _run(tm, torch, Q, K, V, heads, S, d, tm.DTYPE_F32, "hsd", causal, precise, route)
    strided = _run(tm, torch, Q, K, V, heads, S, d, tm.DTYPE_F32, "shd", causal, precise, route)
    typed = _run(tm, torch, Q, K, V, heads, S, d, dtype, "shd", causal, precise, route)[0]
    assert torch.isfinite(ref[0]).all()
    for a, b in zip(ref, strided):
        assert torch.equal(a.view(torch.int8) if a.dtype != torch.int8 else a,
                           b.view(torch.int8) if b.dtype != torch.int8 else b), "strided run differs"
    rounded = ref[0].half() if dtype == tm.DTYPE_F16 else ref[0].bfloat16()
    assert torch.equal(typed.view(torch.int16), rounded.view(torch.int16)), "typed output is not the rounded fp32 O"
