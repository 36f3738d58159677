"""The five BASELINE workloads: shapes, seeded synthetic inputs and routing masks.

Inputs are generated on the device with a seeded torch generator (synthetic
data, [B*H, S, D] contiguous fp16); routing masks are drawn on the host with a
seeded numpy Generator and packed per head into the TileMixRouting word
format (``routing.pack_cells``), with the skip extension where the workload
skips tiles. All routed tiles are whole 64-key groups, so key_tiles_per_group
is 2.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import routing


@dataclass(frozen=True)
class Workload:
    index: int
    name: str
    B: int
    H: int
    S: int
    D: int
    causal: bool
    inputs: str   # "normal" | "outlier" | "student_t"
    router: str   # "bernoulli" | "causal_band" | "importance" | "three_way"
    key_tiles_per_group: int = 2

    @property
    def heads(self) -> int:
        return self.B * self.H

    @property
    def score_scale(self) -> float:
        return float(np.float32(1.0) / np.sqrt(np.float32(self.D)))

    def describe(self) -> str:
        return (f"config{self.index} {self.name}: B={self.B} H={self.H} S={self.S} D={self.D} "
                f"{'causal' if self.causal else 'non-causal'}, inputs={self.inputs}, routing={self.router}")


WORKLOADS = {
    1: Workload(1, "tiny", 1, 4, 256, 64, False, "normal", "bernoulli"),
    2: Workload(2, "mid", 4, 16, 2048, 64, False, "normal", "bernoulli"),
    3: Workload(3, "headline-causal", 4, 16, 4096, 128, True, "normal", "causal_band"),
    4: Workload(4, "long-importance", 1, 32, 16384, 128, False, "outlier", "importance"),
    5: Workload(5, "sparse-three-way", 2, 16, 8192, 128, False, "student_t", "three_way"),
}


def make_inputs(w: Workload, seed: int, device="cuda:0"):
    """Q, K, V as fp16 [B*H, S, D] device tensors.

    normal:    i.i.d. N(0, 1);
    outlier:   N(0, 1) with round(0.02 * D) seeded channels scaled x8 in Q and K;
    student_t: Student-t, nu = 3, divided by sqrt(3) (unit variance).
    """
    import torch

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    shape = (w.heads, w.S, w.D)

    def normal():
        return torch.randn(shape, generator=gen, device=device, dtype=torch.float32)

    if w.inputs == "normal":
        q, k, v = normal(), normal(), normal()
    elif w.inputs == "outlier":
        q, k, v = normal(), normal(), normal()
        count = int(round(0.02 * w.D))
        channels = np.random.default_rng(seed).choice(w.D, size=count, replace=False)
        q[..., channels] *= 8.0
        k[..., channels] *= 8.0
    elif w.inputs == "student_t":
        def student_t():
            z = normal()
            chi2 = normal().square() + normal().square() + normal().square()
            return z / torch.sqrt(chi2 / 3.0) / np.sqrt(3.0)
        q, k, v = student_t(), student_t(), student_t()
    else:
        raise ValueError(w.inputs)
    return tuple(t.to(torch.float16).contiguous() for t in (q, k, v))


def make_codes(w: Workload, seed: int, Q=None, K=None) -> np.ndarray:
    """Per-head cell codes [heads, ceil(S/16), ceil(S/32)] (0 FP16, 1 INT8, 2 skip)."""
    rng = np.random.default_rng(seed + 1)
    codes = []
    if w.router == "importance":
        import torch

        q_amax = Q.view(w.heads, w.S // 128, 128 * w.D).abs().amax(-1).float().cpu().numpy()
        k_amax = K.view(w.heads, w.S // 64, 64 * w.D).abs().amax(-1).float().cpu().numpy()
    for h in range(w.heads):
        if w.router == "bernoulli":
            codes.append(routing.bernoulli_tiles(rng, w.S, w.S, 64, 64))
        elif w.router == "causal_band":
            codes.append(routing.causal_near_diagonal(rng, w.S, 128, 64))
        elif w.router == "importance":
            codes.append(routing.importance_top_fraction(q_amax[h], k_amax[h], w.S, w.S, w.D, 128, 64))
        elif w.router == "three_way":
            codes.append(routing.three_way(rng, w.S, w.S, 64, 64))
        else:
            raise ValueError(w.router)
    return np.stack(codes)


def pack_heads(codes: np.ndarray, key_tiles_per_group: int):
    """Stack per-head packed words: (route_words, skip_words or None), each [heads * words_per_head]."""
    routes, skips = [], []
    for head_codes in codes:
        r, s = routing.pack_cells(head_codes, key_tiles_per_group)
        routes.append(r)
        skips.append(s if s is not None else np.zeros_like(r))
    route_words = np.concatenate(routes)
    skip_words = np.concatenate(skips)
    return route_words, (skip_words if skip_words.any() else None)


def work(w: Workload, codes: np.ndarray) -> dict:
    """Algorithmic ops over all heads, counted from the drawn masks."""
    total = {"ops_int8": 0, "flops_fp16": 0, "pairs_int8": 0, "pairs_fp16": 0}
    for head_codes in codes:
        one = routing.algorithmic_work(head_codes, w.S, w.S, w.D, w.causal)
        total["ops_int8"] += one["ops_int8"]
        total["flops_fp16"] += one["flops_fp16"]
        total["pairs_int8"] += one["pairs"]["int8"]
        total["pairs_fp16"] += one["pairs"]["fp16"]
    return total
