"""The drop-in per-head API at the headline head size.

The restated reference suite (test_reference_suite_gpu.py) runs
quantize_tilemix_qk + launch_fused_fp16_attention on small shapes. Here the
same two calls run once on one head of the headline shape (M = N = 4096,
d = 128, mixed INT8 / FP16 routing with key_tiles_per_group = 2, and the
precise P.V that this API always takes), checked like the reference's own routing cases
(src/tests/tilemix_test.cu:487-500): quantized operands and every INT32 dot
of an INT8 cell bit for bit, the routing trace exactly, and O against the
fp64 TileMix oracle at 1e-5 + 1e-4 |x|. d = 128 runs with O 16-byte aligned
(vector path) and 4-byte aligned (scalar path); d = 64 with the vector path;
M = 4000, N = 4001 puts a partial tile at the end of both (vector path). K and
V are followed by 64 NaN rows in every case, so a read past key N - 1 shows.
"""
import numpy as np
import pytest

from helpers import GUARD_DOT, GUARD_F32, GUARD_TRACE, compare, dev, dev_half, guarded, guarded_lead, host, \
    nan_padded_rows, reference_group_words

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n,d,lead", [(4096, 4096, 128, 4), (4096, 4096, 128, 1), (4096, 4096, 64, 4),
                                        (4000, 4001, 128, 4)],
                         ids=["d128-vector", "d128-scalar", "d64-vector", "ragged-d128-vector"])
def test_per_head_api_headline_size(tm, oracle_lib, cuda, m, n, d, lead):
    import torch

    group = 2
    query_tiles, key_tiles = (m + 15) // 16, (n + 31) // 32
    words, expected_bits = reference_group_words(query_tiles, key_tiles, group, "mixed")
    assert words.size == tm.routing_word_count(m, n, group)
    q, k, v = oracle_lib.make_inputs(m, n, d, "random")
    q8_ref, qs_ref = oracle_lib.quantize(q, 128)
    k8_ref, ks_ref = oracle_lib.quantize(k, 64)
    # K / V followed by 64 NaN rows: a read past key n - 1 would turn into a NaN output.
    dq = dev_half(q)
    dk, dv = dev_half(nan_padded_rows(k.reshape(n, d))), dev_half(nan_padded_rows(v.reshape(n, d)))
    # lead 4: O 16-byte aligned after the guard words (vector path); lead 1: O only 4-byte aligned (scalar path).
    out = guarded_lead(m * d, np.float32, GUARD_F32, fill=np.nan, lead=lead)
    mask = dev(words)
    bits = guarded(expected_bits.size, np.uint8, GUARD_TRACE)
    q8 = torch.empty(q.size, dtype=torch.int8, device="cuda:0")
    k8 = torch.empty(k.size, dtype=torch.int8, device="cuda:0")
    q_scales = torch.empty(qs_ref.size, dtype=torch.int16, device="cuda:0")
    k_scales = torch.empty(ks_ref.size, dtype=torch.int16, device="cuda:0")
    dots = guarded(m * n, np.int32, GUARD_DOT)
    print(f"per-head API M={m} N={n} d={d} g={group} lead={lead} mixed routing", flush=True)
    assert tm.quantize_tilemix_qk(dq, dk, q8, k8, q_scales, k_scales, m, n, d) == tm.SUCCESS
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    routing = tm.TileMixRouting(mask, words.size, group, bits.data_ptr() + 1)
    quantized = tm.TileMixQuantized(q8, k8, q_scales, k_scales, dots.data_ptr() + 4)
    assert tm.launch_fused_fp16_attention(dq, dk, dv, out.data_ptr() + 4 * lead, m, n, d, scale, None,
                                          routing, quantized) == tm.SUCCESS
    torch.cuda.synchronize()

    assert np.array_equal(host(q8), q8_ref.reshape(-1)) and np.array_equal(host(k8), k8_ref.reshape(-1))
    assert np.array_equal(host(q_scales).view(np.uint16), qs_ref)
    assert np.array_equal(host(k_scales).view(np.uint16), ks_ref)
    got_bits = host(bits)
    assert got_bits[0] == GUARD_TRACE and got_bits[-1] == GUARD_TRACE, "routing trace guard overwritten"
    assert np.array_equal(got_bits[1:-1], expected_bits.reshape(-1)), "routing trace differs"
    got_dots = host(dots)
    assert got_dots[0] == GUARD_DOT and got_dots[-1] == GUARD_DOT, "INT32 dot guard overwritten"
    cell_bits = np.repeat(np.repeat(expected_bits, 16, axis=0)[:m], 32, axis=1)[:, :n].astype(bool)
    # |dot| <= 127 * 127 * d < 2^53, so the float64 product is exact.
    exact = (q8_ref.astype(np.float64) @ k8_ref.astype(np.float64).T).astype(np.int64)
    expected_dots = np.where(cell_bits, exact, int(GUARD_DOT)).astype(np.int32)
    mismatch = got_dots[1:-1].reshape(m, n) != expected_dots
    assert not mismatch.any(), f"INT32 dot mismatch at {np.argwhere(mismatch)[:4].tolist()}"

    actual = host(out)
    assert (actual[:lead] == GUARD_F32).all() and actual[-1] == GUARD_F32, "output guard overwritten"
    mixed = oracle_lib.tilemix(q, k, v, q8_ref, k8_ref, qs_ref, ks_ref, expected_bits, scale)
    compare(actual[lead:-1], mixed, 1e-5, 1e-4, "per-head API vs fp64 TileMix oracle")
