"""GPU parity of the quantizer on special values, through the C ABI, against
the C oracle (bit-exact Q8 / K8 / scales).

The reference kernel (src/tilemix.cu:16-49) takes the block maximum with
fmaxf, which skips NaNs, and converts with the saturating __float2int_rz,
which maps a NaN quotient to 0. Blocks here hold NaNs among finite values,
an inf maximum, NaN only, NaN with -inf, -0 only, fp16 subnormals only and
the fp16 maximum, on both sides (128-row Q blocks, 64-row K blocks, ragged
last blocks), for every kernel form: contiguous and row-strided vector
loads at 4 and 8 chunks per thread, and the scalar path (d % 8 != 0).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import dev, dev_half, host

pytestmark = pytest.mark.gpu

NAN, NEG_NAN, INF, NEG_INF, NEG_ZERO = 0x7E00, 0xFE00, 0x7C00, 0xFC00, 0x8000


def special_rows(rows: int, d: int, block: int, rng) -> np.ndarray:
    """[rows, d] fp16 bits: random N(0, 1) with one special pattern per block."""
    x = rng.standard_normal((rows, d)).astype(np.float16).view(np.uint16).copy()
    patterns = ["nan_among", "inf_max", "nan_only", "nan_neg_inf", "neg_zero", "subnormal", "fp16_max", "plain"]
    for b, first in enumerate(range(0, rows, block)):
        last = min(rows, first + block)
        blk = x[first:last]
        kind = patterns[b % len(patterns)]
        r = rng.integers(0, last - first, size=2)
        c = rng.integers(0, d, size=2)
        if kind == "nan_among":
            blk[r[0], c[0]], blk[r[1], c[1]] = NAN, NEG_NAN
        elif kind == "inf_max":
            blk[r[0], c[0]] = INF
        elif kind == "nan_only":
            blk[:] = NAN
        elif kind == "nan_neg_inf":
            blk[r[0], c[0]], blk[r[1], c[1]] = NAN, NEG_INF
            if r[0] == r[1] and c[0] == c[1]:
                blk[(r[0] + 1) % (last - first), c[0]] = NEG_INF
        elif kind == "neg_zero":
            blk[:] = NEG_ZERO
        elif kind == "subnormal":
            blk[:] = rng.integers(1, 0x400, size=blk.shape).astype(np.uint16) | (
                rng.integers(0, 2, size=blk.shape).astype(np.uint16) << 15)
        elif kind == "fp16_max":
            blk[r[0], c[0]] = 0x7BFF
            blk[r[1], c[1]] = 0xFBFF
    return x


def check_side(oracle_lib, x, x8, scales, block, label):
    for h in range(x.shape[0]):
        ref8, ref_scales = oracle_lib.quantize(x[h], block)
        assert np.array_equal(x8[h], ref8), f"{label} bytes head {h}: {np.argwhere(x8[h] != ref8)[:4].tolist()}"
        assert np.array_equal(scales[h], ref_scales), f"{label} scales head {h}: {scales[h]} vs {ref_scales}"


@pytest.mark.parametrize("d", [128, 64, 40, 17])
@pytest.mark.parametrize("mode", ["per_head", "strided", "k_only"])
def test_quantizer_special_values(tm, oracle_lib, cuda, d, mode):
    import torch

    heads, M, N = 3, 300, 200
    rng = np.random.default_rng(1000 * d + len(mode))
    q = np.stack([special_rows(M, d, 128, rng) for _ in range(heads)])
    k = np.stack([special_rows(N, d, 64, rng) for _ in range(heads)])
    q_blocks, k_blocks = (M + 127) // 128, (N + 63) // 64
    Q8 = torch.full((heads, M, d), -128, dtype=torch.int8, device=cuda)
    K8 = torch.full((heads, N, d), -128, dtype=torch.int8, device=cuda)
    qs = torch.full((heads, q_blocks), 0x7B53, dtype=torch.int16, device=cuda)
    ks = torch.full((heads, k_blocks), 0x7B53, dtype=torch.int16, device=cuda)
    print(f"quantizer specials d={d} mode={mode}", flush=True)
    if mode == "per_head":
        Q, K = dev_half(q), dev_half(k)
        for h in range(heads):
            tm.check(tm.quantize_tilemix_qk(Q[h], K[h], Q8[h], K8[h], qs[h], ks[h], M, N, d), "quantize_tilemix_qk")
    else:
        pad = 8
        # Row-strided [rows, heads, d + pad] views: chunks gather across rows.
        q_wide = np.zeros((M, heads, d + pad), dtype=np.uint16)
        k_wide = np.zeros((N, heads, d + pad), dtype=np.uint16)
        q_wide[:, :, :d] = q.transpose(1, 0, 2)
        k_wide[:, :, :d] = k.transpose(1, 0, 2)
        Q, K = dev_half(q_wide), dev_half(k_wide)
        row = heads * (d + pad)
        if mode == "strided":
            tm.check(tm.quantize_tilemix_qk_strided(Q, K, Q8, K8, qs, ks, heads, M, N, d, d + pad, d + pad, row, row),
                     "quantize_tilemix_qk_strided")
        else:
            tm.check(tm.quantize_tilemix_qk_strided(None, K, None, K8, None, ks, heads, M, N, d, 0, d + pad, 0, row),
                     "quantize_tilemix_qk_strided (K only)")
    torch.cuda.synchronize()
    if mode != "k_only":
        check_side(oracle_lib, q, host(Q8), host(qs, np.uint16), 128, "Q")
    else:
        assert (host(Q8) == -128).all() and (host(qs, np.uint16) == 0x7B53).all(), "Q side written in a K-only call"
    check_side(oracle_lib, k, host(K8), host(ks, np.uint16), 64, "K")


@pytest.mark.parametrize("d", [128, 64, 40])
def test_in_kernel_q_quantization_special_values(tm, oracle_lib, cuda, d):
    """quantize=1 of the batched entry point: each workgroup quantizes its
    own 128-row Q block in registers (Q8 / q_scales written out) and the K
    pre-pass writes K8 / k_scales; every cell routed INT8 so both are used."""
    import torch

    heads, M, N = 2, 300, 200
    rng = np.random.default_rng(77 + d)
    q = np.stack([special_rows(M, d, 128, rng) for _ in range(heads)])
    k = np.stack([special_rows(N, d, 64, rng) for _ in range(heads)])
    v = rng.standard_normal((heads, N, d)).astype(np.float16).view(np.uint16)
    words = tm.routing_word_count(M, N, 1)
    route = dev(np.full(heads * words, np.uint64(0xFFFFFFFFFFFFFFFF), dtype=np.uint64))
    O = torch.empty((heads, M, d), dtype=torch.float32, device=cuda)
    Q8 = torch.full((heads, M, d), -128, dtype=torch.int8, device=cuda)
    K8 = torch.full((heads, N, d), -128, dtype=torch.int8, device=cuda)
    qs = torch.full((heads, (M + 127) // 128), 0x7B53, dtype=torch.int16, device=cuda)
    ks = torch.full((heads, (N + 63) // 64), 0x7B53, dtype=torch.int16, device=cuda)
    args = tm.BatchedArgs(Q=dev_half(q), K=dev_half(k), V=dev_half(v), O=O, heads=heads, M=M, N=N, d=d,
                          score_scale=d ** -0.5, quantize=1, route_words=route, key_tiles_per_group=1,
                          Q8=Q8, K8=K8, q_scales=qs, k_scales=ks)
    print(f"in-kernel Q quantization specials d={d}", flush=True)
    tm.check(tm.attention_batched(args), "attention_batched")
    torch.cuda.synchronize()
    check_side(oracle_lib, q, host(Q8), host(qs, np.uint16), 128, "Q (in kernel)")
    check_side(oracle_lib, k, host(K8), host(ks, np.uint16), 64, "K (pre-pass)")
