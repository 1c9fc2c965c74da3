#!/usr/bin/env python3
"""Encoder benchmark: vectors encoded/sec at d=128, M=8, K=256, beam 16 on one MI355X.

Workload (the benchmark's headline configuration): 1M descriptor-like fp32 vectors, d=128,
drawn from a seeded 4096-component Gaussian mixture clipped and rounded to [0,255]; M=8
residual k-means codebooks of K=256; beam width 16; no ICM. One step = one full encode of the
1M vectors already resident in HBM: ||x||^2, xC = C_all^T X (fp32 MFMA), the 8 beam layers, the
LS refit of the coefficients and the per-vector cost (EncodeBase without ICM).

Prints one JSON line. `roofline` covers the dominant kernel (the last beam layer, L=7), priced
by the benchmark's selection-stage figure (4 bytes per scored candidate, 4*K*B per vector per
layer) against HBM; `roofline_distance` covers the xC GEMM (2*d*H flops per vector, lookup
form) against fp32 MFMA. Kernel durations come from HIP events recorded on the stream the
kernels run on. `cpu_baseline` times the CPU oracle (a C++ restatement of the reference
encoder, OpenMP) on the first vectors of the same workload, and `parity` compares the GPU codes
of that sample with the oracle's.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_FP32_MFMA_TFLOPS = 157.3


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--cpu-sample", type=int, default=100_000,
                    help="vectors timed on the CPU oracle (0 = skip)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="after the timed steps, run a plain copy kernel of this many MiB "
                         "(traffic reference for hardware counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the encoder shards by vector range; see the design notes)", file=sys.stderr)
        sys.exit(2)

    from stlq_amd import workloads
    from stlq_amd.encoder import Context, EncodeConfig

    w = workloads.CONFIGS["C2"]
    n = int(args.n)
    t0 = time.perf_counter()
    mix = workloads.Mixture(w.kind, w.d, w.n_comp, w.seed)
    X = mix.sample(0, n)
    C = workloads.make_codebooks(w)
    h = [w.K] * w.m
    log(f"workload generated in {time.perf_counter() - t0:.1f}s: n={n} d={w.d} M={w.m} K={w.K} beam={w.H_beam}")

    ctx = Context(0)
    dev_name, cus = ctx.device_info()
    ctx.set_codebooks(C, h)
    cfg = EncodeConfig(H_beam=w.H_beam, icm_iters=0, want_coeffs=True)
    dX = ctx.dev_alloc(X.nbytes)
    dcodes = ctx.dev_alloc(n * w.m)
    da = ctx.dev_alloc(n * w.m * 4)
    dcost = ctx.dev_alloc(n * 4)
    ctx.h2d(dX, X)

    for k in range(args.warmup):
        ctx.encode_device(dX, n, cfg, dcodes, da, dcost)
        ctx.synchronize()
        log(f"warmup step {k + 1}/{args.warmup} done")

    gemm_ms = beam_ms = total_ms = 0.0
    layer_ms = np.zeros(20)
    launches = 0
    ctx.synchronize()
    t_start = time.perf_counter()
    for k in range(args.steps):
        ctx.encode_device(dX, n, cfg, dcodes, da, dcost)
        t = ctx.last_timings()  # waits for this step's events
        gemm_ms += t.gemm_ms
        beam_ms += t.beam_ms
        total_ms += t.total_ms
        layer_ms += np.array(t.layer_ms[:20])
        launches += t.gemm_launches
    ctx.synchronize()
    wall = time.perf_counter() - t_start
    log(f"timed {args.steps} steps in {wall:.3f}s")

    codes = ctx.d2h(np.empty((n, w.m), np.uint8), dcodes)
    cost = ctx.d2h(np.empty(n, np.float32), dcost)

    if args.calib_copy_mb > 0:
        nb = args.calib_copy_mb * (1 << 20)
        a_ = ctx.dev_alloc(nb)
        b_ = ctx.dev_alloc(nb)
        ctx.lib.stlq_mi355_dev_copy_kernel(ctx.h, a_, b_, nb)
        ctx.synchronize()
        ctx.dev_free(a_)
        ctx.dev_free(b_)
        log(f"calibration copy of {args.calib_copy_mb} MiB done")

    steps = max(args.steps, 1)
    ms_per_step = wall * 1000.0 / steps
    value = n * steps / wall
    K, B, M, d, H = w.K, w.H_beam, w.m, w.d, w.K * w.m
    last = M - 1
    avg_last_ms = layer_ms[last] / steps
    sel_bytes = 4.0 * K * B * n  # scored candidates of one expansion layer
    beam_ach = sel_bytes / (avg_last_ms * 1e-3) / 1e9
    gemm_flops = 2.0 * d * H * n
    avg_gemm_ms = gemm_ms / max(launches, 1)
    gemm_ach = gemm_flops / (avg_gemm_ms * 1e-3) / 1e12
    stages = {
        "gemm_ms": gemm_ms / steps,
        "beam_ms": beam_ms / steps,
        "beam_layer_ms": [round(x / steps, 3) for x in layer_ms[:M]],
        "device_total_ms": total_ms / steps,
    }

    out = {
        "metric": "vectors encoded/sec (d=128,M=8,K=256,B=16)",
        "value": value,
        "unit": "vectors/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "1M descriptor-like vectors d=128 (4096-component GMM, clipped/rounded to [0,255], fp32), "
                        "M=8 x K=256 residual k-means codebooks, beam 16, no ICM, LS refit + cost",
            "n": n, "d": d, "M": M, "K": K, "H_beam": B, "icm_iters": 0,
        },
        "roofline": {
            "kernel": f"beam layer L={last} (LayerKernel<{last}>)",
            "bound": "hbm",
            "achieved": beam_ach,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": beam_ach / PEAK_HBM_GBS,
            "traffic": None,
            "algorithmic_bytes_per_launch": sel_bytes,
            "avg_launch_ms": avg_last_ms,
        },
        "roofline_distance": {
            "kernel": "xC GEMM (GemmXcKernel, fp32 MFMA, lookup form)",
            "bound": "mfma",
            "achieved": gemm_ach,
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": gemm_ach / PEAK_FP32_MFMA_TFLOPS,
            "flops_per_launch": gemm_flops,
            "avg_launch_ms": avg_gemm_ms,
        },
        "stages": stages,
        "device": {"arch": dev_name, "cus": cus},
        "final_mse_mean": float(np.mean(np.maximum(cost.astype(np.float64), 0.0))),
    }

    if args.cpu_sample > 0:
        from oracle import oracle as orc

        ns = min(args.cpu_sample, n)
        threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
        Xs = X[:ns]
        G, inv = orc.build_precomp(C, h, nthreads=threads)
        tc = time.perf_counter()
        nx2 = orc.xnorm2(Xs, nthreads=threads)
        xC = orc.gemm_xc(C, Xs, mode=1, nthreads=threads)
        t_gemm = time.perf_counter() - tc
        codes_o, _ = orc.beam_search(nx2, xC, G, h, B, nthreads=threads)
        t_beam = time.perf_counter() - tc - t_gemm
        a_o, _ = orc.solve_ls_all(xC, G, h, codes_o, nthreads=threads)
        cost_o = orc.compute_costs(xC, G, h, codes_o, a_o, nx2, nthreads=threads)
        t_cpu = time.perf_counter() - tc
        log(f"cpu oracle: {ns} vectors in {t_cpu:.1f}s on {threads} threads")
        cpu_model = ""
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        cpu_model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
        out["cpu_baseline"] = {
            "value": ns / t_cpu,
            "unit": "vectors/s",
            "cores": threads,
            "kind": "port",
            "sample": f"first {ns} vectors of the same workload; ||x||^2 + xC + beam + LS refit + cost; "
                      f"stages s: xC {t_gemm:.2f}, beam {t_beam:.2f}, ls+cost {t_cpu - t_gemm - t_beam:.2f}; "
                      f"cpu: {cpu_model}",
        }
        same = np.all(codes[:ns] == codes_o, axis=1)
        out["parity"] = {
            "sample": ns,
            "codes_identical_frac": float(np.mean(same)),
            "cost_bit_identical_frac": float(np.mean(cost[:ns].view(np.uint32) == cost_o.view(np.uint32))),
        }

    for p in (dX, dcodes, da, dcost):
        ctx.dev_free(p)
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
