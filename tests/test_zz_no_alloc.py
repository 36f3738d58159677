"""The allocation-free importance router (tilemix_tiles_importance_noalloc)
against the workspace entry point it mirrors (tilemix_tiles_importance),
through the C ABI: two calls in a row on the same library scratch, the second
with a smaller problem, each equal byte for byte to the workspace call on the
same inputs. Its size limit and argument checks run without a GPU in
tests/test_capi_cpu.py::test_mask_producer_validation_codes."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _inputs(heads, M, N, d, seed):
    import torch

    g = torch.Generator().manual_seed(seed)
    q = torch.randn((heads, M, d), generator=g).to(torch.float16)
    k = torch.randn((heads, N, d), generator=g).to(torch.float16)
    # A few outlier channels so that tile maxima differ and ties are rare.
    q[:, :, :3] *= 8
    k[:, :, :3] *= 8
    return q.to("cuda:0"), k.to("cuda:0")


def _with_workspace(tm, q, k, heads, M, N, d, tr, tk, fraction):
    import torch

    tiles_q, tiles_k = (M + tr - 1) // tr, (N + tk - 1) // tk
    need = tm.importance_workspace_bytes(heads, M, N, tr, tk)
    ws = torch.empty(need // 4, dtype=torch.float32, device="cuda:0")
    codes = torch.full((heads, tiles_q, tiles_k), 0xEE, dtype=torch.uint8, device="cuda:0")
    tm.check(tm.tiles_importance(q, k, heads, M, N, d, tr, tk, fraction, ws, need, codes), "importance")
    return codes


def test_noalloc_matches_workspace_entry_point(tm, cuda):
    import torch

    assert tm.importance_noalloc_max_bytes() == 1 << 20
    # Config-4-sized first (32 heads, S = 16384, 128 x 64 tiles: 48 KiB of
    # maxima), then a smaller ragged problem on the same scratch.
    for heads, M, N, d, tr, tk, fraction, seed in ((32, 16384, 16384, 128, 128, 64, 0.25, 1),
                                                   (3, 1000, 700, 64, 64, 64, 0.3, 2)):
        print(f"noalloc importance heads={heads} M={M} N={N} d={d} tile={tr}x{tk}", flush=True)
        q, k = _inputs(heads, M, N, d, seed)
        expected = _with_workspace(tm, q, k, heads, M, N, d, tr, tk, fraction)
        codes = torch.full_like(expected, 0xEE)
        tm.check(tm.tiles_importance_noalloc(q, k, heads, M, N, d, tr, tk, fraction, codes), "noalloc importance")
        torch.cuda.synchronize()
        assert torch.equal(codes, expected), f"noalloc codes differ for heads={heads} M={M} N={N}"
        fp16 = int((codes == tm.routing.FP16).sum())
        assert fp16 == heads * int(np.rint(fraction * expected[0].numel())), "FP16 tile count"
