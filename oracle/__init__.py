"""TEST INFRASTRUCTURE - NOT PART OF THE PRODUCT.

ctypes/numpy front end of the C oracle in ``oracle/tilemix_oracle.c`` (a CPU
restatement of the reference's TileMix semantics; per-function reference
citations are in ``tilemix_oracle.h``). Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg import this package, and only as the
checker: the shipped library never calls it.

fp16 tensors are numpy ``uint16`` arrays of IEEE binary16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libtilemix_oracle.so"
_lib = None


def build(force: bool = False) -> Path:
    """Compile the oracle with gcc (``make -C oracle``)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


def _p(array: np.ndarray | None):
    if array is None:
        return None
    assert array.flags.c_contiguous
    return array.ctypes.data_as(ctypes.c_void_p)


def _declare(so: ctypes.CDLL) -> None:
    vp, i32, u32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_size_t
    so.tmo_half_to_float.argtypes = [ctypes.c_uint16]
    so.tmo_half_to_float.restype = ctypes.c_float
    so.tmo_float_to_half.argtypes = [ctypes.c_float]
    so.tmo_float_to_half.restype = ctypes.c_uint16
    so.tmo_halves_to_floats.argtypes = [vp, vp, sz]
    so.tmo_floats_to_halves.argtypes = [vp, vp, sz]
    so.tmo_mt19937_outputs.argtypes = [u32, vp, sz]
    so.tmo_make_inputs.argtypes = [i32, i32, i32, ctypes.c_char_p, vp, vp, vp]
    so.tmo_make_inputs.restype = i32
    so.tmo_quantize.argtypes = [vp, i32, i32, i32, vp, vp]
    so.tmo_int8_dot.argtypes = [vp, vp, i32, i32, i32]
    so.tmo_int8_dot.restype = ctypes.c_int32
    so.tmo_tilemix.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, ctypes.c_float,
                               i32, vp, i32, vp]
    so.tmo_attention.argtypes = [vp, vp, vp, i32, i32, i32, vp]
    so.tmo_attention.restype = i32
    so.tmo_decode_routes.argtypes = [vp, vp, i32, i32, i32, vp]


# ----------------------------------------------------------------- fp16


def half_to_float(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().tmo_halves_to_floats(_p(h), _p(out), h.size)
    return out


def float_to_half(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().tmo_floats_to_halves(_p(f), _p(out), f.size)
    return out


# -------------------------------------------------------------- mt19937


def mt19937_outputs(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint32)
    lib().tmo_mt19937_outputs(seed & 0xFFFFFFFF, _p(out), count)
    return out


# --------------------------------------------------------------- inputs


def make_inputs(m: int, n: int, d: int, pattern: str):
    """Inputs of src/tests/tilemix_test.cu:43-134 as fp16 bit arrays (q, k, v)."""
    q = np.empty((m, d), dtype=np.uint16)
    k = np.empty((n, d), dtype=np.uint16)
    v = np.empty((n, d), dtype=np.uint16)
    status = lib().tmo_make_inputs(m, n, d, pattern.encode(), _p(q), _p(k), _p(v))
    if status != 0:
        raise ValueError(f"pattern {pattern!r} not defined for m={m} n={n} d={d}")
    return q, k, v


# ------------------------------------------------------------ quantizer


def quantize(x: np.ndarray, block_rows: int):
    """reference_tilemix.h:16-41 -> (int8 values [rows, d], fp16 scale bits)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    rows, d = x.shape
    out = np.empty((rows, d), dtype=np.int8)
    scales = np.empty((rows - 1) // block_rows + 1, dtype=np.uint16)
    lib().tmo_quantize(_p(x), rows, d, block_rows, _p(out), _p(scales))
    return out, scales


def int8_dot(q8: np.ndarray, k8: np.ndarray, query: int, key: int) -> int:
    d = q8.shape[1]
    return int(lib().tmo_int8_dot(_p(np.ascontiguousarray(q8)), _p(np.ascontiguousarray(k8)),
                                  query, key, d))


# -------------------------------------------------------------- tilemix


def tilemix(q, k, v, q8=None, k8=None, q_scales=None, k_scales=None, routes=None,
            score_scale: float = 1.0, causal: bool = False, rows=None) -> np.ndarray:
    """reference_tilemix.h:53-90 (+ skip / causal). routes: uint8 [ceil(M/16), ceil(N/32)]."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    M, d = q.shape
    N = k.shape[0]
    if routes is not None:
        routes = np.ascontiguousarray(routes, dtype=np.uint8)
        assert routes.shape == ((M + 15) // 16, (N + 31) // 32)
        if (routes == 1).any():
            assert q8 is not None and k8 is not None and q_scales is not None and k_scales is not None
    row_array = None
    count = M
    if rows is not None:
        row_array = np.ascontiguousarray(rows, dtype=np.int32)
        count = row_array.size
    out = np.empty((count, d), dtype=np.float64)
    conv = lambda a, t: None if a is None else np.ascontiguousarray(a, dtype=t)
    q8, k8 = conv(q8, np.int8), conv(k8, np.int8)
    q_scales, k_scales = conv(q_scales, np.uint16), conv(k_scales, np.uint16)
    lib().tmo_tilemix(_p(q), _p(k), _p(v), _p(q8), _p(k8), _p(q_scales), _p(k_scales),
                      _p(routes), M, N, d, float(score_scale), int(bool(causal)),
                      _p(row_array), count, _p(out))
    return out


def attention(q, k, v) -> np.ndarray:
    """reference_attention.h:12-52: dense fp64 softmax(QK^T/sqrt(d))V."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    M, d = q.shape
    N = k.shape[0]
    out = np.empty((M, d), dtype=np.float64)
    if lib().tmo_attention(_p(q), _p(k), _p(v), M, N, d, _p(out)) != 0:
        raise ValueError("attention requires finite Q/K/V")
    return out


def decode_routes(route_words, skip_words, M: int, N: int, key_tiles_per_group: int) -> np.ndarray:
    routes = np.empty(((M + 15) // 16, (N + 31) // 32), dtype=np.uint8)
    conv = lambda a: None if a is None else np.ascontiguousarray(a, dtype=np.uint64)
    lib().tmo_decode_routes(_p(conv(route_words)), _p(conv(skip_words)), M, N,
                            key_tiles_per_group, _p(routes))
    return routes


def omp_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
