"""GPU parity of the device routing-mask producer (tilemix-cuda_amd/csrc/routing.hip):

* the hash-seeded builders (Bernoulli, causal band, three-way) equal their
  numpy restatement (tests/routing_reference.py) code for code;
* the importance router equals tilemix.routing.importance_top_fraction, ties
  included;
* the packer equals tilemix.routing.pack_cells over cells_from_tiles for
  ragged shapes and key-tile groups of 1 and 2;
* attention over device-built masks equals attention over host-packed masks
  bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

import routing_reference as ref
from tilemix import routing

pytestmark = pytest.mark.gpu

BUILDER_CASES = [  # heads, M, N, tile_rows, tile_keys, seed
    (1, 256, 256, 64, 64, 0),
    (4, 2048, 2048, 64, 64, 17),
    (3, 1000, 777, 128, 64, 5),
    (2, 4096, 4096, 128, 64, 2024),
]


def _codes(torch, heads, M, N, tr, tk):
    tq, tkk = ref.tile_grid(M, N, tr, tk)
    return torch.full((heads, tq, tkk), 0xEE, dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("heads,M,N,tr,tk,seed", BUILDER_CASES)
def test_builders_match_host_restatement(tm, cuda, heads, M, N, tr, tk, seed):
    import torch

    print(f"builders heads={heads} M={M} N={N} tile={tr}x{tk} seed={seed}", flush=True)
    c = _codes(torch, heads, M, N, tr, tk)
    tm.check(tm.tiles_bernoulli(c, heads, M, N, tr, tk, 0.5, seed), "bernoulli")
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), ref.bernoulli(heads, M, N, tr, tk, 0.5, seed))
    c = _codes(torch, heads, M, N, tr, tk)
    tm.check(tm.tiles_three_way(c, heads, M, N, tr, tk, 0.3, 0.4, seed), "three-way")
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), ref.three_way(heads, M, N, tr, tk, 0.3, 0.4, seed))
    c = _codes(torch, heads, M, N, tr, tk)
    tm.check(tm.tiles_three_way(c, heads, M, N, tr, tk, 0.95, 0.03, seed), "three-way, mostly skipped")
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), ref.three_way(heads, M, N, tr, tk, 0.95, 0.03, seed))
    S = M
    c = _codes(torch, heads, S, S, tr, tk)
    tm.check(tm.tiles_causal_band(c, heads, S, tr, tk, 8, 0.5, seed), "causal band")
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), ref.causal_band(heads, S, tr, tk, 8, 0.5, seed))


def _host_importance(q, k, M, N, d, tr, tk, fraction):
    """Per-tile maxima from the same fp16 data, then the host router (tile codes)."""
    tq, tkk = ref.tile_grid(M, N, tr, tk)
    def amax(block):  # NaN elements passed over, as fmaxf from 0 does
        a = np.abs(block.astype(np.float32))
        return np.where(np.isnan(a), np.float32(0), a).max()

    qa = np.array([amax(q[i * tr:(i + 1) * tr]) for i in range(tq)])
    ka = np.array([amax(k[j * tk:(j + 1) * tk]) for j in range(tkk)])
    cells = routing.importance_top_fraction(qa, ka, M, N, d, tr, tk, fraction)
    return cells[:: tr // 16, :: tk // 32][:tq, :tkk]


@pytest.mark.parametrize("heads,M,N,d,tr,tk,fraction,pattern", [
    (2, 2048, 2048, 128, 128, 64, 0.25, "outlier"),
    (3, 1000, 1500, 64, 64, 64, 0.3, "normal"),
    (2, 1024, 1024, 128, 128, 64, 0.25, "ties"),
    (1, 512, 512, 32, 128, 64, 0.0, "normal"),
    (1, 512, 512, 32, 128, 64, 1.0, "normal"),
    (4, 16384, 16384, 128, 128, 64, 0.25, "outlier"),
    (2, 700, 900, 36, 64, 64, 0.4, "normal"),  # d % 8 != 0: the element-wise maximum
    (2, 1000, 1200, 64, 64, 64, 0.3, "nan"),
    (2, 4096, 4096, 64, 64, 64, 0.37, "ties"),  # ties ranked across several 1024-tile chunks
    (1, 3000, 50, 32, 16, 64, 0.5, "normal"),  # one key tile per row
    (1, 130, 70000, 64, 64, 64, 0.3, "ties"),  # rows longer than the select's 1024 threads
    (1, 2048, 4096, 16, 16, 32, 0.4, "ties"),  # 16384 tiles: keys held in registers, ties ranked
    (2, 1000, 5000, 16, 16, 32, 0.3, "normal"),  # 9891 tiles: a ragged last wave of register keys
    (1, 1000, 5000, 16, 16, 32, 0.75, "zeros"),  # selected key 0, tied with the ragged padding
    (1, 4096, 8192, 16, 16, 32, 0.45, "ties"),  # 65536 tiles: keys recomputed each pass
    # tiles_q + tiles_k = 15360 + 1024 = 16384, the select's LDS limit (64 KiB of factors)
    (1, 16 * 15360, 32 * 1024, 16, 16, 32, 0.25, "outlier"),
])
def test_importance_matches_host_router(tm, cuda, heads, M, N, d, tr, tk, fraction, pattern):
    import torch

    print(f"importance heads={heads} M={M} N={N} d={d} tile={tr}x{tk} fraction={fraction} {pattern}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(M + N + d)
    q = torch.randn(heads, M, d, generator=g, device="cuda")
    k = torch.randn(heads, N, d, generator=g, device="cuda")
    if pattern == "outlier":
        ch = torch.tensor([3, 17, 40][: max(1, d // 48)], device="cuda")
        q[..., ch] *= 8.0
        k[..., ch] *= 8.0
    if pattern == "zeros":  # half the query tiles all zero: many keys equal to 0
        q[:, : M // 2] = 0.0
    if pattern == "ties":  # many equal tile maxima: ranks decided by tile index
        q = torch.round(q * 2) / 2
        k = torch.round(k * 2) / 2
        q.clamp_(-2, 2)
        k.clamp_(-2, 2)
    q, k = q.half().contiguous(), k.half().contiguous()
    if pattern == "nan":  # scattered NaNs, and one Q tile and one K tile that are all NaN
        q[:, 5, 3] = float("nan")
        q[:, 300, :] = float("nan")
        q[:, tr:2 * tr, :] = float("nan")
        k[:, 7, 0] = float("nan")
        k[:, (N - 1) // tk * tk:, :] = float("nan")
    tq, tkk = ref.tile_grid(M, N, tr, tk)
    need = tm.importance_workspace_bytes(heads, M, N, tr, tk)
    ws = torch.empty(need // 4, dtype=torch.float32, device="cuda")
    c = _codes(torch, heads, M, N, tr, tk)
    tm.check(tm.tiles_importance(q, k, heads, M, N, d, tr, tk, fraction, ws, need, c), "importance")
    torch.cuda.synchronize()
    got = c.cpu().numpy()
    qn, kn = q.cpu().numpy(), k.cpu().numpy()
    for h in range(heads):
        expected = _host_importance(qn[h], kn[h], M, N, d, tr, tk, fraction)
        assert np.array_equal(got[h], expected), f"head {h}"
        assert int((got[h] == routing.FP16).sum()) == int(round(fraction * tq * tkk))


@pytest.mark.parametrize("M,N,tr,tk,g", [
    (256, 256, 64, 64, 2), (256, 256, 64, 64, 1), (1000, 777, 128, 64, 2), (1000, 777, 16, 32, 1),
    (4096, 4096, 128, 64, 2), (300, 5000, 48, 96, 3), (17, 33, 16, 32, 1),
])
def test_pack_matches_host_packer(tm, cuda, M, N, tr, tk, g):
    import torch

    heads = 3
    print(f"pack M={M} N={N} tile={tr}x{tk} g={g}", flush=True)
    tq, tkk = ref.tile_grid(M, N, tr, tk)
    rng = np.random.default_rng(M * 31 + N)
    codes = rng.integers(0, 3, size=(heads, tq, tkk), dtype=np.uint8)
    wc = tm.routing_word_count(M, N, g)
    route = torch.full((heads * wc,), -1, dtype=torch.int64, device="cuda")
    skip = torch.full((heads * wc,), -1, dtype=torch.int64, device="cuda")
    c = torch.from_numpy(codes).to("cuda")
    tm.check(tm.routes_from_tiles(c, heads, M, N, tr, tk, g, route, skip), "pack")
    torch.cuda.synchronize()
    r = route.cpu().numpy().view(np.uint64).reshape(heads, wc)
    s = skip.cpu().numpy().view(np.uint64).reshape(heads, wc)
    for h in range(heads):
        er, es = routing.pack_cells(routing.cells_from_tiles(codes[h], tr, tk, M, N), g)
        assert np.array_equal(r[h], er), f"route words head {h}"
        assert np.array_equal(s[h], es if es is not None else np.zeros_like(er)), f"skip words head {h}"


def test_attention_over_device_masks_equals_host_masks(tm, cuda):
    import torch
    from tilemix import workloads

    heads, S, D, tr, tk, g = 4, 1024, 64, 64, 64, 2
    print(f"attention over device masks heads={heads} S={S} D={D}", flush=True)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(9)
    Q, K, V = (torch.randn(heads, S, D, generator=gen, device="cuda").half() for _ in range(3))
    c = _codes(torch, heads, S, S, tr, tk)
    tm.check(tm.tiles_three_way(c, heads, S, S, tr, tk, 0.3, 0.4, 77), "three-way")
    wc = tm.routing_word_count(S, S, g)
    route = torch.empty(heads * wc, dtype=torch.int64, device="cuda")
    skip = torch.empty(heads * wc, dtype=torch.int64, device="cuda")
    tm.check(tm.routes_from_tiles(c, heads, S, S, tr, tk, g, route, skip), "pack")
    torch.cuda.synchronize()
    codes = c.cpu().numpy()
    host_route, host_skip = [], []
    for h in range(heads):
        r, s = routing.pack_cells(routing.cells_from_tiles(codes[h], tr, tk, S, S), g)
        host_route.append(r)
        host_skip.append(s if s is not None else np.zeros_like(r))
    outs = []
    for rw, sw in ((route, skip),
                   (torch.from_numpy(np.concatenate(host_route).view(np.int64)).cuda(),
                    torch.from_numpy(np.concatenate(host_skip).view(np.int64)).cuda())):
        O = torch.empty(heads, S, D, device="cuda")
        K8 = torch.empty(heads, S, D, dtype=torch.int8, device="cuda")
        ks = torch.empty(heads, S // 64, dtype=torch.int16, device="cuda")
        args = tm.BatchedArgs(Q=Q, K=K, V=V, O=O, heads=heads, M=S, N=S, d=D, score_scale=D ** -0.5,
                              quantize=1, route_words=rw, skip_words=sw, key_tiles_per_group=g, K8=K8,
                              k_scales=ks)
        tm.check(tm.attention_batched(args), "attention")
        torch.cuda.synchronize()
        outs.append(O.cpu())
    assert torch.equal(outs[0], outs[1])
    assert torch.isfinite(outs[0]).all()
