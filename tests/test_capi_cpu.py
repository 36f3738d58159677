"""The C-ABI library without a GPU: it loads, exports exactly what
include/tilemix_capi.h declares, answers the sizing helpers, and returns the
reference's validation codes before any HIP runtime call
(src/tests/tilemix_test.cu:157-234 is the list of cases), and the product never
reaches the oracle. The native program's CPU mode is run by
tests/test_native_export.py.
"""
from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import tilemix
from tilemix import api

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tilemix_capi.h"
INVALID, NOT_SUPPORTED = api.ERROR_INVALID_VALUE, api.ERROR_NOT_SUPPORTED
INT_MAX = 2 ** 31 - 1


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^(?:int|size_t|const char\s*\*)\s+(tilemix_\w+)\s*\(", text, re.M))


def test_library_loads_and_reports_version(tm):
    assert tm.version().startswith("tilemix-hip") and "gfx950" in tm.version()


def test_every_declared_symbol_is_exported(tm):
    lib = tm.library()
    declared = declared_symbols()
    assert {"tilemix_quantize_qk", "tilemix_attention", "tilemix_attention_batched",
            "tilemix_quantize_qk_batched"} <= declared
    for name in declared:
        assert hasattr(lib, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", str(api.library_path())], check=True,
                        capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in nm.splitlines() if " T " in line and "tilemix_" in line}
    assert exported == declared, f"undeclared exports {exported - declared}, missing {declared - exported}"


def test_sizing_helpers_known_values(tm):
    # src/tests/tilemix_test.cu:186-191 (shared-memory footprints of the reference layout)
    assert tm.shared_bytes(1, False) == 4608
    assert tm.shared_bytes(17, False) == 7168
    assert tm.shared_bytes(128, False) == 22528
    assert tm.shared_bytes(129, False) == 0
    assert tm.shared_bytes(128, True) == 28672
    assert tm.shared_bytes(17, True) == 8704
    # :208-217
    assert tm.routing_word_count(17, 2048, 1) == 2
    assert tm.routing_word_count(17, 2049, 1) == 4
    assert tm.routing_word_count(17, 4097, 2) == 4
    assert tm.routing_word_count(17, 4097, 1) == 6
    assert tm.routing_word_count(17, INT_MAX, INT_MAX) == 2
    assert tm.routing_word_count(0, 1, 1) == 0
    assert tm.routing_word_count(1, 0, 1) == 0
    assert tm.routing_word_count(1, 1, 0) == 0
    assert tm.routing_words_per_row(4097, 1) == 3 and tm.routing_words_per_row(1, 0) == 0


class HostArgs:
    """Host addresses: valid as pointers for argument validation, never dereferenced."""

    def __init__(self):
        self.x = np.ones(4, dtype=np.float16)
        self.out = np.zeros(4, dtype=np.float32)
        self.byte = np.zeros(4, dtype=np.int8)
        self.scale = np.zeros(4, dtype=np.float16)
        self.word = np.zeros(4, dtype=np.uint64)

    def p(self, a):
        return a.ctypes.data


def test_attention_validation_codes(tm):
    h = HostArgs()
    x, o = h.p(h.x), h.p(h.out)
    attn = tm.launch_fused_fp16_attention
    assert attn(None, x, x, o, 1, 1, 1, 1.0) == INVALID
    assert attn(x, None, x, o, 1, 1, 1, 1.0) == INVALID
    assert attn(x, x, None, o, 1, 1, 1, 1.0) == INVALID
    assert attn(x, x, x, None, 1, 1, 1, 1.0) == INVALID
    for bad in (0, -1):
        assert attn(x, x, x, o, bad, 1, 1, 1.0) == INVALID
        assert attn(x, x, x, o, 1, bad, 1, 1.0) == INVALID
        assert attn(x, x, x, o, 1, 1, bad, 1.0) == INVALID
    for d in (129, INT_MAX):
        assert attn(x, x, x, o, 1, 1, d, 1.0) == NOT_SUPPORTED
    for scale in (float("nan"), float("inf"), float("-inf")):
        assert attn(x, x, x, o, 1, 1, 1, scale) == INVALID
    partial = tilemix.TileMixQuantized(q=h.p(h.byte))
    assert attn(x, x, x, o, 1, 1, 1, 1.0, quantized=partial) == INVALID
    for group in (0, -1):
        assert attn(x, x, x, o, 1, 1, 1, 1.0, routing=tilemix.TileMixRouting(None, 0, group)) == INVALID
    word = h.p(h.word)
    assert attn(x, x, x, o, 1, 1, 1, 1.0, routing=tilemix.TileMixRouting(word, 1, 1)) == INVALID
    for routing in (tilemix.TileMixRouting(None, 1, 1), tilemix.TileMixRouting(word, 0, 1),
                    tilemix.TileMixRouting(word, 3, 1)):
        assert attn(x, x, x, o, 17, 2049, 1, 1.0, routing=routing) == INVALID


def test_quantizer_validation_codes(tm):
    h = HostArgs()
    x, b, s = h.p(h.x), h.p(h.byte), h.p(h.scale)
    quant = tm.quantize_tilemix_qk
    assert quant(None, x, b, b, s, s, 1, 1, 1) == INVALID
    assert quant(x, x, None, b, s, s, 1, 1, 1) == INVALID
    assert quant(x, x, b, b, None, s, 1, 1, 1) == INVALID
    assert quant(x, x, b, b, s, s, 0, 1, 1) == INVALID
    assert quant(x, x, b, b, s, s, 1, 1, 129) == NOT_SUPPORTED
    batched = tm.quantize_tilemix_qk_batched
    assert batched(x, x, b, b, s, s, 0, 1, 1, 1) == INVALID
    assert batched(x, x, b, b, s, s, 2, 4, 4, 4, q_head_stride=8) == INVALID   # stride < M*d


def test_batched_validation_codes(tm):
    h = HostArgs()
    x, o, b, s, w = h.p(h.x), h.p(h.out), h.p(h.byte), h.p(h.scale), h.p(h.word)

    def run(**kw):
        base = dict(Q=x, K=x, V=x, O=o, heads=1, M=1, N=1, d=1, score_scale=1.0, quantize=0)
        base.update(kw)
        return tm.attention_batched(tilemix.BatchedArgs(**base))

    assert tm.library().tilemix_attention_batched(None, None) == INVALID
    assert run(Q=None) == INVALID
    assert run(heads=0) == INVALID
    assert run(M=-1) == INVALID
    assert run(d=129) == NOT_SUPPORTED
    assert run(score_scale=float("nan")) == INVALID
    assert run(heads=2, M=4, d=4, q_head_stride=8) == INVALID
    assert run(quantize=3) == INVALID
    assert run(route_words=w, key_tiles_per_group=0) == INVALID
    assert run(route_words=w) == INVALID                       # INT8 routes without K8
    assert run(route_words=w, K8=b, k_scales=s) == INVALID     # quantize=0 needs Q8 and q_scales
    assert run(route_words=w, K8=b, k_scales=s, quantize=2, Q8=b) == INVALID  # Q8 without q_scales
    assert run(score_dots=w) == INVALID                        # dots need INT8 routes
    # layout and output options
    assert run(o_dtype=3) == INVALID
    assert run(o_dtype=-1) == INVALID
    assert run(d=4, q_row_stride=3) == INVALID                 # rows closer than d
    assert run(d=4, o_row_stride=2) == INVALID
    # heads interleaved in rows too short to hold them all overlap
    assert run(heads=2, M=4, N=4, d=4, q_head_stride=4, k_head_stride=4, v_head_stride=4, o_head_stride=4,
               q_row_stride=8, k_row_stride=8, v_row_stride=8, o_row_stride=6) == INVALID
    assert run(heads=3, M=4, N=4, d=4, q_head_stride=4, k_head_stride=4, v_head_stride=4, o_head_stride=4,
               q_row_stride=8, k_row_stride=8, v_row_stride=8, o_row_stride=8) == INVALID
    strided = tm.quantize_tilemix_qk_strided
    assert strided(x, x, b, b, s, s, 1, 4, 4, 4, q_row_stride=2) == INVALID
    assert strided(x, x, b, b, s, s, 2, 4, 4, 4, q_head_stride=4, k_head_stride=16, q_row_stride=6) == INVALID
    assert strided(x, x, b, b, s, s, 1, 4, 4, 129) == NOT_SUPPORTED


def test_mask_producer_validation_codes(tm):
    """The device mask producer rejects bad arguments before any HIP call."""
    fake = 0x1000  # never dereferenced: every case below fails validation first
    # packer: null pointers, sizes, tile shapes, a key-tile group straddling two tiles
    assert tm.routes_from_tiles(None, 1, 64, 64, 64, 64, 2, fake, fake) == INVALID
    assert tm.routes_from_tiles(fake, 1, 64, 64, 64, 64, 2, None, fake) == INVALID
    assert tm.routes_from_tiles(fake, 1, 64, 64, 64, 64, 2, fake, None) == INVALID
    assert tm.routes_from_tiles(fake, 0, 64, 64, 64, 64, 2, fake, fake) == INVALID
    assert tm.routes_from_tiles(fake, 1, 0, 64, 64, 64, 2, fake, fake) == INVALID
    assert tm.routes_from_tiles(fake, 1, 64, 64, 24, 64, 2, fake, fake) == INVALID   # not whole 16-row cells
    assert tm.routes_from_tiles(fake, 1, 64, 64, 64, 48, 1, fake, fake) == INVALID   # not whole 32-key cells
    assert tm.routes_from_tiles(fake, 1, 64, 64, 64, 32, 2, fake, fake) == INVALID   # group of 2 spans 2 tiles
    assert tm.routes_from_tiles(fake, 1, 64, 64, 64, 96, 2, fake, fake) == INVALID   # 3 cells per tile, g = 2
    assert tm.routes_from_tiles(fake, 1, 64, 64, 64, 64, 0, fake, fake) == INVALID
    # builders: probabilities, band, shapes
    assert tm.tiles_bernoulli(fake, 1, 64, 64, 64, 64, 1.5, 0) == INVALID
    assert tm.tiles_bernoulli(fake, 1, 64, 64, 64, 64, float("nan"), 0) == INVALID
    assert tm.tiles_bernoulli(None, 1, 64, 64, 64, 64, 0.5, 0) == INVALID
    assert tm.tiles_causal_band(fake, 1, 64, 128, 64, -1, 0.5, 0) == INVALID
    assert tm.tiles_causal_band(fake, 1, 0, 128, 64, 8, 0.5, 0) == INVALID
    assert tm.tiles_three_way(fake, 1, 64, 64, 64, 64, 0.7, 0.4, 0) == INVALID   # p_skip + p_int8 > 1
    assert tm.tiles_three_way(fake, 1, 64, 64, 64, 64, -0.1, 0.4, 0) == INVALID
    # importance router: workspace sizing and checks
    assert tm.importance_workspace_bytes(32, 16384, 16384, 128, 64) == 32 * (128 + 256) * 4
    assert tm.importance_workspace_bytes(0, 16384, 16384, 128, 64) == 0
    need = tm.importance_workspace_bytes(2, 256, 256, 128, 64)
    assert tm.tiles_importance(fake, fake, 2, 256, 256, 64, 128, 64, 0.25, fake, need - 1, fake) == INVALID
    assert tm.tiles_importance(fake, fake, 2, 256, 256, 64, 128, 64, 1.25, fake, need, fake) == INVALID
    assert tm.tiles_importance(None, fake, 2, 256, 256, 64, 128, 64, 0.25, fake, need, fake) == INVALID
    assert tm.tiles_importance(fake, fake, 2, 256, 256, 64, 128, 64, 0.25, fake, need, fake,
                               q_head_stride=100) == INVALID                        # overlapping heads
    huge = tm.importance_workspace_bytes(1, 16 * 20000, 64, 16, 64)
    assert tm.tiles_importance(fake, fake, 1, 16 * 20000, 64, 64, 16, 64, 0.25, fake, huge, fake) == NOT_SUPPORTED
    # allocation-free importance router: its fixed scratch bounds the problem
    assert tm.importance_noalloc_max_bytes() == 1 << 20
    assert tm.importance_workspace_bytes(1024, 16384, 16384, 128, 64) > tm.importance_noalloc_max_bytes()
    assert tm.tiles_importance_noalloc(fake, fake, 1024, 16384, 16384, 128, 128, 64, 0.25, fake) == INVALID
    assert tm.tiles_importance_noalloc(None, fake, 2, 256, 256, 64, 128, 64, 0.25, fake) == INVALID
    assert tm.tiles_importance_noalloc(fake, fake, 2, 256, 256, 64, 128, 64, 1.25, fake) == INVALID
    assert tm.tiles_importance_noalloc(fake, fake, 2, 256, 256, 64, 128, 64, 0.25, None) == INVALID
    assert tm.tiles_importance_noalloc(fake, fake, 2, 256, 256, 64, 128, 64, 0.25, fake,
                                       q_head_stride=100) == INVALID                # overlapping heads
    assert tm.tiles_importance_noalloc(fake, fake, 1, 16 * 20000, 64, 64, 16, 64, 0.25, fake) == NOT_SUPPORTED


def test_missing_library_fails_loudly(tmp_path):
    # A copy of the binding package with no library beside it: it must raise,
    # not fall back to anything.
    shutil.copytree(ROOT / "tilemix-cuda_amd" / "tilemix", tmp_path / "pkg" / "tilemix")
    code = ("import sys; sys.path.insert(0, %r)\n"
            "import tilemix\n"
            "assert not tilemix.library_path().exists()\n"
            "try:\n    tilemix.library()\nexcept ImportError as e:\n    print('ImportError', e)\n"
            % str(tmp_path / "pkg"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert "ImportError" in out.stdout and "no fallback" in out.stdout, out.stderr


def test_product_never_uses_the_oracle():
    package = ROOT / "tilemix-cuda_amd"
    offenders = []
    for path in package.rglob("*"):
        if path.suffix in (".py", ".hip", ".h", ".cpp") and "_build" not in path.parts:
            text = path.read_text(errors="replace")
            if re.search(r"\bimport oracle\b|from oracle\b|tilemix_oracle|libtilemix_oracle", text):
                offenders.append(str(path.relative_to(ROOT)))
    assert not offenders, offenders
    deps = subprocess.run(["ldd", str(api.library_path())], capture_output=True, text=True).stdout
    assert "oracle" not in deps
