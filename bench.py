#!/usr/bin/env python3
"""Fused-QKV RNS GEMM + reconstruction on one MI355X.

Workload (the metric's config): fused OPT-125m QKV,
K=768, N=3x768=2304, R=4 channels (255, 253, 251, 247), M=256 tokens.
Weights: per-output-channel symmetric int8 of seeded N(0, 0.02) matrices;
activations: per-token int8 of seeded N(0, 1).  One step = one
``matmul_prepared_fused`` call (residue encode + MFMA GEMM + reduction +
Garner + signed correction, exact int64 output) with inputs resident in HBM.
The prepared weights rotate over copies totalling more than 512 MB so the
256 MB MALL cannot serve repeats.

Printed JSON (one line): value = effective int8 TOPS = 2*R*M*K*N / t_step;
roofline of the dominant kernel (the GEMM) timed alone with HIP events;
cpu_baseline = the NumPy restatement of the reference CPU path on a bounded
sample, 1 core.  Extra rows cover the other C2 token counts, C3 decode and
a C5 (OPT-6.7B QKV) shape.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rns-llm_amd"))
sys.path.insert(0, ROOT)

DENSE4 = (255, 253, 251, 247)
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # dense int8 MFMA, MI355X


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def quant_rows_int8(w):
    import torch

    amax = w.abs().amax(dim=1, keepdim=True)
    scale = torch.clamp(amax / 127.0, min=torch.finfo(torch.float32).eps)
    return torch.clamp(torch.round(w / scale), -127, 127).to(torch.int8)


def make_weights(backend, k, n_each, parts, count, seed, device):
    """`count` prepared fused weights (B^T = [parts*n_each, k]) and their int8."""
    import torch

    gen = torch.Generator(device=device).manual_seed(seed)
    prepared, raw = [], []
    for i in range(count):
        blocks = [quant_rows_int8(torch.randn((n_each, k), generator=gen, device=device,
                                              dtype=torch.float32).half().float() * 0.02)
                  for _ in range(parts)]
        w = torch.cat(blocks, dim=0).contiguous()           # [N, K] int8
        prepared.append(backend.prepare_weight_nk(w, DENSE4))
        if i == 0:
            raw.append(w)
    return prepared, raw[0]


def make_tokens(m, k, seed, device):
    import torch

    gen = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn((m, k), generator=gen, device=device)
    return quant_rows_int8(x).contiguous()


def exact_check(out, a, w_nk, max_rows=256):
    """Bit-exact check against the closed-form int64 product (all rows up to
    max_rows, an evenly spaced subset beyond)."""
    import torch

    rows = torch.arange(a.shape[0])
    if a.shape[0] > max_rows:
        rows = torch.linspace(0, a.shape[0] - 1, max_rows).long()
    want = a.cpu()[rows].to(torch.int64) @ w_nk.cpu().to(torch.int64).t()
    if not torch.equal(out.cpu()[rows], want):
        bad = int((out.cpu()[rows] != want).sum())
        raise SystemExit(f"parity failure: {bad} outputs differ from the exact int64 product")


def time_loop(fn, steps, warmup):
    import torch

    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms


def per_call(fn, iters):
    import torch

    samples = []
    for i in range(iters):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn(i)
        e.record()
        e.synchronize()
        samples.append(s.elapsed_time(e) * 1000.0)
    samples.sort()
    return statistics.median(samples), samples[min(len(samples) - 1, math.ceil(0.95 * len(samples)) - 1)]


def measure_shape(backend, name, m, k, n_each, parts, steps, warmup, rotate_bytes, seed, device,
                  check=True):
    import torch

    n = n_each * parts
    r = len(DENSE4)
    res_bytes = r * n * ((k + 63) // 64 * 64)
    count = max(2, math.ceil(rotate_bytes / res_bytes))
    prepared, w0 = make_weights(backend, k, n_each, parts, count, seed, device)
    a = make_tokens(m, k, seed + 1, device)
    ws = backend.create_workspace(device=device, channels=r, m=m, n=n, k=k)
    out0 = backend.matmul_prepared_fused(a, prepared[0], workspace=ws).clone()
    if check:
        exact_check(out0, a, w0, max_rows=256 if k * n < 4_000_000 else 16)

    def step(i):
        backend.matmul_prepared_fused(a, prepared[i % count], workspace=ws)

    ms = time_loop(step, steps, warmup)
    p50, p95 = per_call(step, min(200, max(50, steps)))

    # dominant kernel alone: GEMM on pre-encoded residues, same rotation
    a_res = backend.encode_activations(a, prepared[0])
    out = torch.empty((m, n), dtype=torch.int64, device=device)

    def gemm(i):
        backend.matmul_residues_prepared(a_res, prepared[i % count], out=out)

    gemm_ms = time_loop(gemm, steps, warmup)
    if check and not torch.equal(backend.matmul_residues_prepared(a_res, prepared[0], out=out), out0):
        raise SystemExit("parity failure: GEMM-only path differs from the fused call")
    ops = 2 * r * m * k * n
    bytes_alg = m * k + r * k * n + m * n * 8
    t_roof = max(ops / (INT8_PEAK_TOPS * 1e12), bytes_alg / (HBM_PEAK_GBS * 1e9))
    row = {
        "config": name, "m": m, "k": k, "n": n, "channels": r, "weight_copies": count,
        "ms_per_step": ms, "us_per_call_p50": p50, "us_per_call_p95": p95,
        "eff_tops": ops / (ms * 1e-3) / 1e12, "useful_tops": ops / r / (ms * 1e-3) / 1e12,
        "gemm_kernel_us": gemm_ms * 1000.0,
        "gemm_hbm_gbs": bytes_alg / (gemm_ms * 1e-3) / 1e9,
        "gemm_eff_tops": ops / (gemm_ms * 1e-3) / 1e12,
        "roofline_frac_step": t_roof / (ms * 1e-3),
        "roofline_frac_gemm": t_roof / (gemm_ms * 1e-3),
        "bound": "hbm" if bytes_alg / (HBM_PEAK_GBS * 1e9) >= ops / (INT8_PEAK_TOPS * 1e12) else "mfma",
        "ops_eff": ops, "bytes_alg": bytes_alg,
    }
    del prepared, ws, a_res, out
    torch.cuda.empty_cache()
    return row


def cpu_baseline(seconds):
    """NumPy restatement of the reference CPU pipeline on a C2 sample."""
    import numpy as np

    from oracle import rns_oracle

    rng = np.random.default_rng(5)
    m, k, n = 16, 768, 2304
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    b = rng.integers(-127, 128, (k, n)).astype(np.int8)
    rns_oracle.rns_matmul_centered(a, b, DENSE4)  # warmup
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        rns_oracle.rns_matmul_centered(a, b, DENSE4)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    ops = 2 * len(DENSE4) * m * k * n
    return {
        "value": ops / t / 1e12, "unit": "effective int8 TOPS", "cores": 1, "kind": "port",
        "sample": (f"C2 slice M={m}, K={k}, N={n}, R=4: NumPy int64 centered encode -> "
                   f"per-channel matmul -> mod -> Garner (oracle/rns_oracle.py), median of "
                   f"{len(times)} calls, {t * 1e3:.1f} ms/call; host {platform.processor() or platform.machine()}, "
                   f"os.cpu_count()={os.cpu_count()}"),
    }


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--m", type=int, default=256)
    parser.add_argument("--rotate-mb", type=float, default=600.0)
    parser.add_argument("--cpu-seconds", type=float, default=10.0)
    parser.add_argument("--no-extra", action="store_true", help="headline shape only")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the RNS path has no "
              "collective, see DESIGN.md for how it would shard", file=sys.stderr)
        sys.exit(2)

    import torch

    from rns_llm_amd import HipRNSBackend

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    backend = HipRNSBackend()
    rot = int(args.rotate_mb * 1e6)
    log(f"bench: C2 fused QKV M={args.m} K=768 N=2304 R=4, steps={args.steps} warmup={args.warmup}")
    head = measure_shape(backend, "C2 fused QKV", args.m, 768, 768, 3, args.steps, args.warmup, rot,
                         17, device)
    log(f"bench: headline {head['us_per_call_p50']:.2f} us/call, {head['eff_tops']:.1f} eff TOPS, "
        f"GEMM {head['gemm_kernel_us']:.2f} us")
    rows = [head]
    if not args.no_extra:
        for m in (1, 16, 128):
            rows.append(measure_shape(backend, "C2 fused QKV", m, 768, 768, 3, args.steps,
                                      args.warmup, rot, 17, device))
            log(f"bench: C2 M={m} {rows[-1]['us_per_call_p50']:.2f} us/call")
        for req in (1, 2, 4):
            rows.append(measure_shape(backend, f"C3 decode {req} requests", req, 768, 768, 1,
                                      args.steps, args.warmup, rot, 33, device))
            log(f"bench: C3 {req} req {rows[-1]['us_per_call_p50']:.2f} us/call")
        for m in (1, 512):
            rows.append(measure_shape(backend, "C5 OPT-6.7B QKV", m, 4096, 4096, 3,
                                      max(20, args.steps // 4), max(5, args.warmup // 4),
                                      rot, 67, device))
            log(f"bench: C5 M={m} {rows[-1]['us_per_call_p50']:.2f} us/call, "
                f"{rows[-1]['eff_tops']:.1f} eff TOPS")

    cpu = cpu_baseline(args.cpu_seconds)
    gemm_s = head["gemm_kernel_us"] * 1e-6
    achieved = head["bytes_alg"] / gemm_s / 1e9
    line = {
        "metric": "effective int8 TOPS + us/call, fused-QKV RNS GEMM+reconstruct, bit-exact",
        "value": head["eff_tops"],
        "unit": "effective int8 TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "us_per_call_p50": head["us_per_call_p50"],
        "us_per_call_p95": head["us_per_call_p95"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) tokens, int8-quantized)",
        "config": {"workload": "C2 fused OPT-125m QKV: M=256, K=768, N=2304, R=4 "
                               "(255,253,251,247), int64 exact output, weights rotated over "
                               f"{head['weight_copies']} copies (> 512 MB)",
                   "m": args.m, "k": 768, "n": 2304, "channels": 4},
        "roofline": {"bound": head["bound"], "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "gemm (rnsmx_matmul_residues_prepared)",
                     "kernel_us": head["gemm_kernel_us"]},
        "cpu_baseline": cpu,
        "rows": rows,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
