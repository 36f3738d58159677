"""TEST INFRASTRUCTURE - NOT PART OF THE PRODUCT.

CPU PyTorch counterpart of the reference's CPU path
(python/reference_attention.py:11-25): dense softmax(Q K^T / sqrt(d)) V in
float32 (or float64) on CPU tensors. It is the ``cpu_baseline`` leg of
bench.py (timed on the GPU host's cores) and a cross-check in tests; nothing
in the library calls it.

Extensions for the bench workloads, not in the reference: ``causal`` (key k
visible to query q only when k <= q) and ``key_mask`` (boolean [M, N], False
= masked); masked scores are -inf before the softmax. ``scale`` overrides
1/sqrt(d) when given.
"""
from __future__ import annotations

import math

import torch


def reference_attention(q, k, v, *, compute_dtype=torch.float32, causal=False, key_mask=None, scale=None):
    if compute_dtype not in (torch.float32, torch.float64):
        raise ValueError("compute_dtype must be torch.float32 or torch.float64")
    for tensor in (q, k, v):
        if tensor.device.type != "cpu" or tensor.ndim != 2 or not tensor.is_contiguous():
            raise ValueError("expected contiguous rank-2 CPU tensors")
        if tensor.dtype not in (torch.float16, torch.float32, torch.float64):
            raise ValueError("expected floating-point tensors")
        if not torch.isfinite(tensor).all().item():
            raise ValueError("expected finite inputs")
    m, d = q.shape
    n = k.shape[0]
    if m <= 0 or d <= 0 or n <= 0 or k.shape[1] != d or v.shape != k.shape:
        raise ValueError("expected Q[M,d], K[N,d], V[N,d] with positive dimensions")
    factor = (1.0 / math.sqrt(d)) if scale is None else scale
    scores = (q.to(compute_dtype) @ k.to(compute_dtype).T) * factor
    if causal:
        scores = scores.masked_fill(torch.ones(m, n, dtype=torch.bool).triu(1), float("-inf"))
    if key_mask is not None:
        scores = scores.masked_fill(~key_mask, float("-inf"))
    return torch.softmax(scores, dim=-1) @ v.to(compute_dtype)
