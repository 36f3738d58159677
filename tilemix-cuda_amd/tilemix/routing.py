"""Host-side routing masks in the TileMixRouting word format.

Word format (reference include/attention_fused.h:34-52, decode in
src/tilemix.cu:99-103): one bit per group of ``key_tiles_per_group``
consecutive 32-key tiles, 64 groups per uint64 word, ``words_per_row`` words
per 16-row query tile; bit 1 = INT8 scores, 0 = FP16. The skip extension uses
a second word array with the same packing (bit 1 = skip).

Cell codes used throughout: 0 = FP16, 1 = INT8, 2 = skip, one per
(16-row query tile, 32-key tile) cell.

The builders for the BASELINE workloads express their coarser tiles
(64x64, 128x64) by replicating a tile's code over the 16x32 cells it covers.
"""
from __future__ import annotations

import numpy as np

CELL_ROWS = 16
CELL_KEYS = 32
FP16, INT8, SKIP = 0, 1, 2


def words_per_row(N: int, key_tiles_per_group: int) -> int:
    if N <= 0 or key_tiles_per_group <= 0:
        return 0
    key_tiles = (N - 1) // CELL_KEYS + 1
    groups = (key_tiles - 1) // key_tiles_per_group + 1
    return (groups - 1) // 64 + 1


def word_count(M: int, N: int, key_tiles_per_group: int) -> int:
    if M <= 0:
        return 0
    return ((M - 1) // CELL_ROWS + 1) * words_per_row(N, key_tiles_per_group)


def cell_grid(M: int, N: int) -> tuple[int, int]:
    return (M + CELL_ROWS - 1) // CELL_ROWS, (N + CELL_KEYS - 1) // CELL_KEYS


def pack_group_bits(group_bits: np.ndarray) -> np.ndarray:
    """[query_tiles, groups] booleans -> uint64 words [query_tiles * words_per_row]."""
    bits = np.asarray(group_bits, dtype=bool)
    rows, groups = bits.shape
    wpr = (groups + 63) // 64
    padded = np.zeros((rows, wpr * 64), dtype=np.uint64)
    padded[:, :groups] = bits
    weights = np.left_shift(np.uint64(1), np.arange(64, dtype=np.uint64))
    words = (padded.reshape(rows, wpr, 64) * weights).sum(axis=2, dtype=np.uint64)
    return np.ascontiguousarray(words.reshape(-1))


def pack_cells(codes: np.ndarray, key_tiles_per_group: int = 1):
    """Cell codes [query_tiles, key_tiles] -> (route_words, skip_words or None).

    Every group of ``key_tiles_per_group`` key tiles must carry one code per row.
    """
    codes = np.asarray(codes, dtype=np.uint8)
    rows, key_tiles = codes.shape
    g = key_tiles_per_group
    groups = (key_tiles - 1) // g + 1
    padded = np.empty((rows, groups * g), dtype=np.uint8)
    padded[:, :key_tiles] = codes
    padded[:, key_tiles:] = codes[:, -1:]  # the ragged last group repeats its own code
    grouped = padded.reshape(rows, groups, g)
    if not (grouped == grouped[:, :, :1]).all():
        raise ValueError("cell codes are not constant within each key-tile group")
    first = grouped[:, :, 0]
    route_words = pack_group_bits(first == INT8)
    skip_words = pack_group_bits(first == SKIP) if (first == SKIP).any() else None
    return route_words, skip_words


def cells_from_tiles(tile_codes: np.ndarray, tile_rows: int, tile_keys: int, M: int, N: int) -> np.ndarray:
    """Replicate codes of tile_rows x tile_keys tiles over the 16x32 cells they cover."""
    if tile_rows % CELL_ROWS or tile_keys % CELL_KEYS:
        raise ValueError("tiles must be whole routing cells")
    rows, cols = cell_grid(M, N)
    tile_codes = np.asarray(tile_codes, dtype=np.uint8)
    row_tile = np.arange(rows) // (tile_rows // CELL_ROWS)
    col_tile = np.arange(cols) // (tile_keys // CELL_KEYS)
    return np.ascontiguousarray(tile_codes[np.ix_(row_tile, col_tile)])


def tile_grid(M: int, N: int, tile_rows: int, tile_keys: int) -> tuple[int, int]:
    return (M + tile_rows - 1) // tile_rows, (N + tile_keys - 1) // tile_keys


# --------------------------------------------------------------- BASELINE masks


def bernoulli_tiles(rng: np.random.Generator, M: int, N: int, tile_rows: int = 64, tile_keys: int = 64,
                    p_int8: float = 0.5) -> np.ndarray:
    """Configs 1-2: per (query tile, key tile) INT8 with probability p_int8, else FP16."""
    tq, tk = tile_grid(M, N, tile_rows, tile_keys)
    tiles = (rng.random((tq, tk)) < p_int8).astype(np.uint8)
    return cells_from_tiles(tiles, tile_rows, tile_keys, M, N)


def causal_near_diagonal(rng: np.random.Generator, S: int, tile_rows: int = 128, tile_keys: int = 64,
                         fp16_band: int = 8, p_int8: float = 0.5) -> np.ndarray:
    """Config 3: causal 128x64 tiles. Tiles entirely above the diagonal are skipped;
    the ``fp16_band`` key tiles ending at the diagonal tile are forced FP16; the rest are
    INT8 with probability p_int8. Tile (i, j) is above the diagonal when its first key
    exceeds the tile's last query row."""
    tq, tk = tile_grid(S, S, tile_rows, tile_keys)
    i = np.arange(tq)[:, None]
    j = np.arange(tk)[None, :]
    last_visible = (i * tile_rows + tile_rows - 1) // tile_keys  # last key tile touching row block i
    draws = (rng.random((tq, tk)) < p_int8).astype(np.uint8)
    tiles = np.where(j > last_visible, SKIP, np.where(last_visible - j < fp16_band, FP16, draws))
    return cells_from_tiles(tiles.astype(np.uint8), tile_rows, tile_keys, S, S)


def importance_top_fraction(q_absmax: np.ndarray, k_absmax: np.ndarray, M: int, N: int, d: int,
                            tile_rows: int = 128, tile_keys: int = 64, fp16_fraction: float = 0.25) -> np.ndarray:
    """Config 4: per tile, the |q.k| bound d * amax_Q(tile) * amax_K(tile); the top
    fp16_fraction of tiles (ties broken by tile index) go FP16, the rest INT8."""
    estimate = d * np.outer(np.asarray(q_absmax, np.float64), np.asarray(k_absmax, np.float64))
    flat = estimate.reshape(-1)
    count = int(round(fp16_fraction * flat.size))
    order = np.lexsort((np.arange(flat.size), -flat))  # descending estimate, then index
    tiles = np.full(flat.size, INT8, dtype=np.uint8)
    tiles[order[:count]] = FP16
    return cells_from_tiles(tiles.reshape(estimate.shape), tile_rows, tile_keys, M, N)


def three_way(rng: np.random.Generator, M: int, N: int, tile_rows: int = 64, tile_keys: int = 64,
              p_skip: float = 0.3, p_int8: float = 0.4) -> np.ndarray:
    """Config 5: per tile skip / INT8 / FP16 with probabilities p_skip / p_int8 / rest;
    a query tile left entirely skipped gets one random tile forced FP16."""
    tq, tk = tile_grid(M, N, tile_rows, tile_keys)
    u = rng.random((tq, tk))
    tiles = np.where(u < p_skip, SKIP, np.where(u < p_skip + p_int8, INT8, FP16)).astype(np.uint8)
    for row in np.nonzero((tiles == SKIP).all(axis=1))[0]:
        tiles[row, rng.integers(tk)] = FP16
    return cells_from_tiles(tiles, tile_rows, tile_keys, M, N)


# ------------------------------------------------------------------ work model


def pair_counts(codes: np.ndarray, M: int, N: int, causal: bool) -> dict:
    """Visible (query, key) pairs per route, counted exactly from the cell codes."""
    rows, cols = codes.shape
    q_lo = np.arange(rows) * CELL_ROWS
    q_hi = np.minimum(q_lo + CELL_ROWS, M)
    k_lo = np.arange(cols) * CELL_KEYS
    k_hi = np.minimum(k_lo + CELL_KEYS, N)
    if causal:
        # pairs with key <= query inside the cell: sum over queries of clip(q + 1 - k_lo, 0, width)
        counts = np.zeros((rows, cols), dtype=np.int64)
        for r in range(rows):
            qs = np.arange(q_lo[r], q_hi[r])[:, None]
            counts[r] = np.clip(qs + 1 - k_lo[None, :], 0, (k_hi - k_lo)[None, :]).sum(axis=0)
    else:
        counts = np.outer(q_hi - q_lo, k_hi - k_lo).astype(np.int64)
    return {
        "int8": int(counts[codes == INT8].sum()),
        "fp16": int(counts[codes == FP16].sum()),
        "skip": int(counts[codes == SKIP].sum()),
    }


def algorithmic_work(codes: np.ndarray, M: int, N: int, d: int, causal: bool, heads: int = 1) -> dict:
    """Ops of one pass: QK^T = 2d per visible pair (INT8 or FP16 by route) and
    P.V = 2d fp16 flops per visible pair; skipped/masked pairs count nothing."""
    pairs = pair_counts(codes, M, N, causal)
    ops_i8 = 2 * d * pairs["int8"] * heads
    flops_f16 = (2 * d * pairs["fp16"] + 2 * d * (pairs["int8"] + pairs["fp16"])) * heads
    return {"ops_int8": ops_i8, "flops_fp16": flops_f16, "pairs": pairs}
