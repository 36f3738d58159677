"""TileMix fused attention benchmark on one MI355X.

Default workload: BASELINE config 3 (the headline): B=4 H=16 S=4096 D=128,
causal, 128x64 routing tiles (above-diagonal tiles skipped, the 8 key tiles
nearest the diagonal FP16, the rest INT8 with p=0.5), inputs N(0,1) fp16.

One step = the whole TileMix job on inputs already resident in HBM:
  1. tilemix_quantize_qk_batched on K (64-row blocks -> K8 + k_scales), then
  2. tilemix_attention_batched with quantize=2 (each workgroup quantizes its own
     128-row Q block in registers, routes every 16x32 cell to INT8 or FP16 MFMA
     or skip, online softmax, P.V on FP16 MFMA, fp32 O).
``value`` = effective TFLOP/s of the step: algorithmic ops counted from the
drawn mask (QK^T 2D per visible pair as INT8 or FP16 by route, P.V 2D FP16)
over the wall time of K steps. ``roofline`` covers the attention kernel alone:
its average duration from HIP events on its stream, against the blended
INT8/FP16 MFMA peak of the same op mix. ``cpu_baseline`` times the CPU PyTorch
restatement of the reference's CPU path (python/reference_attention.py) on a
bounded sample of heads on this host's cores.

Warm-up: the W requested steps, then more untimed steps until at least
--min-warmup-ms of wall time has passed since warm-up began. An MI355X
raises its clock over the first tens of milliseconds of sustained work (the
headline attention launch goes from about 0.39 ms to 0.31 ms after roughly
50 ms), so a few steps alone would time the ramp rather than the sustained
rate. The JSON line reports W as requested and the steps actually run; the
timed region is exactly K steps either way.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--min-warmup-ms T] [--config 3]
                       [--precise] [--no-check] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tilemix-cuda_amd"))

PEAK_FP16_TFLOPS = 2516.6   # MI355X dense FP16 MFMA (256 CU x 2.4 GHz x 4096 flop/clk)
PEAK_INT8_TOPS = 5033.2     # MI355X dense INT8 MFMA
PEAK_HBM_GBS = 8000.0


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--min-warmup-ms", type=float, default=150.0,
                   help="keep running untimed steps after the W warm-up steps until this much wall "
                        "time has passed since warm-up began (0 disables)")
    p.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5])
    p.add_argument("--seed", type=int, default=20261201)
    p.add_argument("--precise", action="store_true", help="split-precision P.V (fp32-level accuracy)")
    p.add_argument("--no-check", action="store_true", help="skip the parity check against the oracle")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU-baseline work")
    p.add_argument("--check-rows", type=int, default=4096)
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="after timing, run one device copy of this many MiB on the bench stream "
                        "(calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE against known bytes)")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the TileMix path shards across "
                          "GPUs by head with no exchange (see DESIGN.md), but multi-GPU runs are not "
                          "part of this build; run with --gpus 1"}))
        return 2

    import torch
    import tilemix
    from tilemix import workloads

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    torch.cuda.set_device(0)
    w = workloads.WORKLOADS[args.config]
    log(w.describe())
    Q, K, V = workloads.make_inputs(w, args.seed)
    codes = workloads.make_codes(w, args.seed, Q, K)
    route_np, skip_np = workloads.pack_heads(codes, w.key_tiles_per_group)
    work = workloads.work(w, codes)
    heads, S, D = w.heads, w.S, w.D
    dev = "cuda:0"
    route_words = torch.from_numpy(route_np.view(np.int64)).to(dev)
    skip_words = torch.from_numpy(skip_np.view(np.int64)).to(dev) if skip_np is not None else None
    O = torch.empty((heads, S, D), dtype=torch.float32, device=dev)
    K8 = torch.empty((heads, S, D), dtype=torch.int8, device=dev)
    k_scales = torch.empty((heads, (S + 63) // 64), dtype=torch.int16, device=dev)
    stream = torch.cuda.Stream()
    attn_args = tilemix.BatchedArgs(Q=Q, K=K, V=V, O=O, heads=heads, M=S, N=S, d=D,
                                    score_scale=w.score_scale, causal=w.causal, precise=args.precise,
                                    quantize=2, route_words=route_words, skip_words=skip_words,
                                    key_tiles_per_group=w.key_tiles_per_group, K8=K8, k_scales=k_scales)

    def step(events=None):
        tilemix.check(tilemix.quantize_tilemix_qk_batched(None, K, None, K8, None, k_scales, heads, S, S, D,
                                                          stream=stream), "quantize K")
        if events is not None:
            events[0].record(stream)
        tilemix.check(tilemix.attention_batched(attn_args, stream), "attention")
        if events is not None:
            events[1].record(stream)

    with torch.cuda.stream(stream):
        warm_start = time.perf_counter()
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        warmup_run = args.warmup
        while (time.perf_counter() - warm_start) * 1e3 < args.min_warmup_ms and warmup_run < 100000:
            for _ in range(8):
                step()
            warmup_run += 8
            torch.cuda.synchronize()
        warmup_ms = (time.perf_counter() - warm_start) * 1e3
        log(f"warm-up: {warmup_run} steps in {warmup_ms:.1f} ms ({args.warmup} requested, "
            f"minimum {args.min_warmup_ms:g} ms)")
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for _ in range(args.steps)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(args.steps):
            step(pairs[k])
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        if args.copy_probe_mib > 0:
            src = torch.ones(args.copy_probe_mib << 19, dtype=torch.float16, device=dev)
            dst = torch.empty_like(src)
            torch.cuda.synchronize()
            dst.copy_(src)
            torch.cuda.synchronize()
            log(f"copy probe: {args.copy_probe_mib} MiB read + {args.copy_probe_mib} MiB written")
            del src, dst
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    attn_ms = float(np.mean([a.elapsed_time(b) for a, b in pairs]))
    log(f"step {ms_per_step:.4f} ms, attention kernel {attn_ms:.4f} ms (HIP events)")

    ops_total = work["ops_int8"] + work["flops_fp16"]
    t_min = work["ops_int8"] / (PEAK_INT8_TOPS * 1e12) + work["flops_fp16"] / (PEAK_FP16_TFLOPS * 1e12)
    blended_peak = ops_total / t_min / 1e12
    achieved = ops_total / (attn_ms * 1e-3) / 1e12
    value = ops_total / (ms_per_step * 1e-3) / 1e12

    result = {
        "metric": "effective TFLOP/s & % MFMA peak, TileMix attn B=4 H=16 S=4096 D=128",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warmup_run,
        "warmup_ms": round(warmup_ms, 1),
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8+f16 (i32/f32 accumulate)",
        "data": "synthetic (seeded torch N(0,1)/outlier/Student-t fp16; seeded numpy routing masks)",
        "config": {
            "workload": w.describe(),
            "B": w.B, "H": w.H, "S": S, "D": D, "causal": w.causal,
            "key_tiles_per_group": w.key_tiles_per_group,
            "precise_pv": bool(args.precise),
            "visible_pairs_int8": work["pairs_int8"], "visible_pairs_fp16": work["pairs_fp16"],
            "ops_int8": work["ops_int8"], "flops_fp16": work["flops_fp16"],
            "step": "K pre-pass quantizer + attention (Q quantized in-kernel)",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "attention_kernel",
            "achieved": round(achieved, 3),
            "peak": round(blended_peak, 3),
            "unit": "TFLOP/s",
            "frac": round(achieved / blended_peak, 4),
            "traffic": None,
            "kernel_ms": round(attn_ms, 5),
            "achieved_hbm_gbs": None,
            "peak_basis": "blended: ops_int8/5033.2T + flops_fp16/2516.6T",
        },
    }

    measured = measured_traffic(w.describe())
    if measured is not None:
        result["roofline"]["traffic"] = measured["traffic_bytes"]
        result["roofline"]["achieved_hbm_gbs"] = round(measured["traffic_bytes"] / (attn_ms * 1e-3) / 1e9, 1)
        result["roofline"]["traffic_source"] = measured["source"]

    if not args.no_check:
        result["parity"] = parity_check(w, Q, K, V, O, K8, k_scales, codes, args)
        log(f"parity: {result['parity']}")

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, Q, K, V, codes, args.cpu_budget)
        log(f"cpu baseline: {result['cpu_baseline']}")

    print(json.dumps(result), flush=True)
    return 0


def measured_traffic(workload: str):
    """HBM bytes per attention launch measured with rocprofv3 FETCH_SIZE/WRITE_SIZE
    (calibrated on a copy of known size) for this workload, if recorded."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    entry = json.loads(path.read_text()).get("attention_kernel")
    return entry if entry and entry.get("workload") == workload else None


def parity_check(w, Q, K, V, O, K8, k_scales, codes, args) -> dict:
    """K8/k_scales bit-exact vs the oracle quantizer (all heads); O vs the fp64
    oracle on a seeded sample of (head, row) pairs: max-abs <= 2e-3, mean-abs <= 2e-4."""
    import torch
    sys.path.insert(0, str(ROOT))
    import oracle

    oracle.build()
    heads, S, D = w.heads, w.S, w.D
    to_bits = lambda t: t.detach().cpu().view(torch.int16).numpy().view(np.uint16)
    q_all, k_all, v_all = to_bits(Q), to_bits(K), to_bits(V)
    k8_all = K8.cpu().numpy()
    ks_all = k_scales.cpu().numpy().view(np.uint16)
    o_all = O.cpu().numpy()
    rng = np.random.default_rng(args.seed + 7)
    sample_heads = sorted(set(rng.choice(heads, size=min(heads, 4), replace=False).tolist()))
    rows_per_head = max(1, args.check_rows // len(sample_heads))
    k8_exact = True
    max_abs, sum_abs, count = 0.0, 0.0, 0
    for h in range(heads):
        k8_ref, ks_ref = oracle.quantize(k_all[h], 64)
        k8_exact &= bool(np.array_equal(k8_ref, k8_all[h]) and np.array_equal(ks_ref, ks_all[h]))
    for h in sample_heads:
        q8_ref, qs_ref = oracle.quantize(q_all[h], 128)
        k8_ref, ks_ref = oracle.quantize(k_all[h], 64)
        rows = np.sort(rng.choice(S, size=min(S, rows_per_head), replace=False)).astype(np.int32)
        expected = oracle.tilemix(q_all[h], k_all[h], v_all[h], q8_ref, k8_ref, qs_ref, ks_ref, codes[h],
                                  w.score_scale, w.causal, rows=rows)
        err = np.abs(o_all[h][rows].astype(np.float64) - expected)
        max_abs = max(max_abs, float(err.max()))
        sum_abs += float(err.sum())
        count += err.size
    mean_abs = sum_abs / count
    return {"k8_kscales_bit_exact": k8_exact, "sampled_heads": sample_heads, "sampled_rows": count // D,
            "max_abs": max_abs, "mean_abs": mean_abs,
            "pass": bool(k8_exact and max_abs <= 2e-3 and mean_abs <= 2e-4)}


def cpu_baseline(w, Q, K, V, codes, budget_s: float) -> dict:
    """CPU PyTorch restatement of python/reference_attention.py on whole heads of the
    same workload until ``budget_s`` seconds of work; throughput over the sampled heads."""
    import torch
    sys.path.insert(0, str(ROOT))
    from oracle.torch_reference import reference_attention
    from tilemix import routing

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    q_cpu, k_cpu, v_cpu = (t.cpu() for t in (Q, K, V))
    rows, cols = codes.shape[1:]

    def key_mask(h):
        if not (codes[h] == routing.SKIP).any():
            return None
        cell = np.repeat(np.repeat(codes[h] != routing.SKIP, 16, axis=0)[: w.S], 32, axis=1)[:, : w.S]
        return torch.from_numpy(np.ascontiguousarray(cell))

    with torch.inference_mode():
        reference_attention(q_cpu[0][:64].contiguous(), k_cpu[0][:64].contiguous(), v_cpu[0][:64].contiguous())
        done, ops, t_total = 0, 0, 0.0
        while done < w.heads and t_total < budget_s:
            mask = key_mask(done)
            t0 = time.perf_counter()
            reference_attention(q_cpu[done], k_cpu[done], v_cpu[done], causal=w.causal, key_mask=mask,
                                scale=w.score_scale)
            t_total += time.perf_counter() - t0
            one = routing.algorithmic_work(codes[done], w.S, w.S, w.D, w.causal)
            ops += one["ops_int8"] + one["flops_fp16"]
            done += 1
    return {"value": round(ops / t_total / 1e12, 5), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"{done} of {w.heads} heads (full S={w.S}), torch {torch.__version__} CPU fp32 dense "
                      f"softmax attention (python/reference_attention.py restated, masked scores -inf), "
                      f"{t_total:.2f} s, cpu '{model}'",
            "seconds": round(t_total, 3), "heads": done}


if __name__ == "__main__":
    sys.exit(main())
