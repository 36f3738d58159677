"""Host restatement of the device mask producer's random builders (test
helper): the counter-based draws of tilemix-cuda_amd/csrc/routing.hip in
numpy uint64 arithmetic, and the builders' rules on top of them. The packer
and the importance router are checked against tilemix.routing
(pack_cells / importance_top_fraction) instead.
"""
from __future__ import annotations

import numpy as np

FP16, INT8, SKIP = 0, 1, 2
_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(x) -> np.ndarray:
    """splitmix64 output for state x (the state is advanced by the golden gamma first)."""
    with np.errstate(over="ignore"):
        z = np.asarray(x, dtype=np.uint64) + _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform24(seed: int, index, salt: int) -> np.ndarray:
    """The device draw: top 24 bits of splitmix64(seed ^ splitmix64(2 * index + salt)) / 2^24, as float32."""
    with np.errstate(over="ignore"):
        inner = splitmix64(np.asarray(index, dtype=np.uint64) * np.uint64(2) + np.uint64(salt))
    h = splitmix64(np.uint64(seed) ^ inner)
    return (h >> np.uint64(40)).astype(np.float32) * np.float32(1.0 / 16777216.0)


def tile_grid(M: int, N: int, tile_rows: int, tile_keys: int) -> tuple[int, int]:
    return (M + tile_rows - 1) // tile_rows, (N + tile_keys - 1) // tile_keys


def linear_index(heads: int, tq: int, tk: int) -> np.ndarray:
    return np.arange(heads * tq * tk, dtype=np.uint64).reshape(heads, tq, tk)


def bernoulli(heads, M, N, tile_rows, tile_keys, p_int8, seed) -> np.ndarray:
    tq, tk = tile_grid(M, N, tile_rows, tile_keys)
    u = uniform24(seed, linear_index(heads, tq, tk), 0)
    return np.where(u < np.float32(p_int8), INT8, FP16).astype(np.uint8)


def causal_band(heads, S, tile_rows, tile_keys, fp16_band, p_int8, seed) -> np.ndarray:
    tq, tk = tile_grid(S, S, tile_rows, tile_keys)
    u = uniform24(seed, linear_index(heads, tq, tk), 0)
    i = np.arange(tq)[None, :, None]
    j = np.arange(tk)[None, None, :]
    last = (i * tile_rows + tile_rows - 1) // tile_keys
    draw = np.where(u < np.float32(p_int8), INT8, FP16)
    return np.where(j > last, SKIP, np.where(last - j < fp16_band, FP16, draw)).astype(np.uint8)


def three_way(heads, M, N, tile_rows, tile_keys, p_skip, p_int8, seed) -> np.ndarray:
    tq, tk = tile_grid(M, N, tile_rows, tile_keys)
    u = uniform24(seed, linear_index(heads, tq, tk), 0)
    bound = np.float32(np.float32(p_skip) + np.float32(p_int8))
    codes = np.where(u < np.float32(p_skip), SKIP, np.where(u < bound, INT8, FP16)).astype(np.uint8)
    rows = codes.reshape(heads * tq, tk)
    for r in np.nonzero((rows == SKIP).all(axis=1))[0]:
        with np.errstate(over="ignore"):
            h = splitmix64(np.uint64(seed) ^ splitmix64(np.uint64(2) * np.uint64(r) + np.uint64(1)))
        rows[r, int(h % np.uint64(tk))] = FP16
    return rows.reshape(heads, tq, tk)
