"""Test helpers: host/device transfer of fp16 bit arrays, guards, comparisons.

Device memory comes from torch (plumbing only); all computation under test goes
through the C ABI of libtilemix_hip.so.
"""
from __future__ import annotations

import numpy as np

GUARD_F32 = np.float32(-12345.25)  # src/tests/tilemix_test.cu:273
GUARD_I8 = np.int8(-128)            # 0x80 fill, tilemix_test.cu:394
GUARD_SCALE = np.uint16(0x7B53)     # fp16(60000), tilemix_test.cu:397
GUARD_TRACE = np.uint8(0xA5)        # tilemix_test.cu:468
GUARD_DOT = np.int32(0x2468ACE)     # tilemix_test.cu:476


def torch_mod():
    import torch

    return torch


def dev_half(bits: np.ndarray):
    """uint16 fp16 bit array -> torch.float16 device tensor."""
    torch = torch_mod()
    host = torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16))
    return host.view(torch.float16).to("cuda:0")


def dev(array: np.ndarray):
    torch = torch_mod()
    array = np.ascontiguousarray(array)
    if array.dtype == np.uint64:
        return torch.from_numpy(array.view(np.int64)).to("cuda:0")
    if array.dtype == np.uint16:
        return torch.from_numpy(array.view(np.int16)).to("cuda:0")
    return torch.from_numpy(array).to("cuda:0")


def host(tensor, dtype=None) -> np.ndarray:
    torch = torch_mod()
    t = tensor.detach().to("cpu")
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().view(np.uint16)
    out = t.numpy()
    return out.view(dtype) if dtype is not None else out


def guarded(count: int, dtype, guard, fill=None):
    """Device buffer of count + 2 elements: guard, fill..., guard."""
    buffer = np.full(count + 2, guard if fill is None else fill, dtype=dtype)
    buffer[0] = buffer[-1] = guard
    return dev(buffer)


def guarded_lead(count: int, dtype, guard, fill=None, lead: int = 1):
    """Device buffer of lead + count + 1 elements: `lead` guards, fill..., guard.
    The payload starts lead * itemsize bytes in: lead = 1 for a 4-byte element
    gives an output that is not 16-byte aligned (the kernels' element-wise
    path), lead = 4 one that is (their 16-byte vector path)."""
    buffer = np.full(count + lead + 1, guard if fill is None else fill, dtype=dtype)
    buffer[:lead] = guard
    buffer[-1] = guard
    return dev(buffer)


def nan_padded_rows(bits: np.ndarray, rows: int = 64) -> np.ndarray:
    """A [n, d] fp16 bit array followed by `rows` rows of NaN (0x7E00): a
    kernel that reads past row n - 1 (up to the end of its last 64-key tile)
    turns the NaN into a NaN output, since 0 * NaN = NaN in P.V."""
    bits = np.asarray(bits, dtype=np.uint16)
    return np.concatenate([bits, np.full((rows,) + bits.shape[1:], 0x7E00, dtype=np.uint16)])


def compare(actual: np.ndarray, expected: np.ndarray, atol: float, rtol: float, label: str) -> dict:
    """|a - e| <= atol + rtol |e| elementwise (src/tests/tilemix_test.cu:137-155)."""
    actual = np.asarray(actual, dtype=np.float64).reshape(-1)
    expected = np.asarray(expected, dtype=np.float64).reshape(-1)
    assert actual.shape == expected.shape and actual.size > 0, label
    error = np.abs(actual - expected)
    finite = np.isfinite(actual) & np.isfinite(expected)
    bad = ~finite | (error > atol + rtol * np.abs(expected))
    if bad.any():
        index = int(np.nonzero(bad)[0][0])
        raise AssertionError(f"{label}: mismatch at {index}: got {actual[index]!r} expected "
                             f"{expected[index]!r} ({int(bad.sum())} of {bad.size} outside tolerance)")
    return {"max_abs": float(error.max()),
            "max_rel": float((error / np.maximum(np.abs(expected), atol)).max()),
            "rms": float(np.sqrt((error ** 2).mean()))}


def reference_group_words(query_tiles: int, key_tiles: int, group: int, pattern: str):
    """Independent mask packer of src/tests/tilemix_test.cu:432-448: logical group
    decisions first, expanded to per-tile bits without dividing by the group size.
    Returns (words uint64, expected per-cell bits uint8)."""
    groups = (key_tiles + group - 1) // group
    wpr = (groups + 63) // 64
    words = [0xFFFFFFFFFFFFFFFF] * (query_tiles * wpr)
    bits = np.zeros((query_tiles, key_tiles), dtype=np.uint8)
    for row in range(query_tiles):
        tile = 0
        for grp in range(groups):
            bit = pattern == "int8-requested" or (pattern == "mixed" and (grp + row + grp // 64) % 2 == 0)
            flag = 1 << (grp % 64)
            index = row * wpr + grp // 64
            words[index] = (words[index] | flag) if bit else (words[index] & ~flag & 0xFFFFFFFFFFFFFFFF)
            repeat = 0
            while repeat < group and tile < key_tiles:
                bits[row, tile] = bit
                repeat += 1
                tile += 1
    return np.array(words, dtype=np.uint64), bits
