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
kernels run on. `cpu_baseline` times the reference's own CPU encoder, compiled from its sources
into oracle/_ref (kind "reference"), or the CPU oracle (a C++ restatement of it, kind "port")
where that build is absent, on the first vectors of the same workload with all host threads;
`parity` compares the GPU codes of that sample with the same CPU run's.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_FP32_MFMA_TFLOPS = 157.3
# VALU issue ceiling: a wave64 fp32 VALU instruction occupies one 16-lane SIMD for 4 cycles; 4 SIMDs
# per CU, 256 CUs, 2.4 GHz peak engine clock. With packed fp32 disabled this is the vector fp32
# rate of 78.6 TFLOP/s (FMA), half of the packed 157.3.
PEAK_VALU_WAVE_INSTS = 256 * 4 * 2.4e9 / 4


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _profile_table(name: str):
    """Rows of the first markdown table in profiles/<name> as {kernel: {column: value}}."""
    path = os.path.join(ROOT, "profiles", name)
    rows, head = {}, None
    try:
        with open(path) as f:
            for line in f:
                if not line.startswith("|"):
                    if head is not None and rows:
                        break
                    continue
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if head is None:
                    head = cells
                elif not set(cells[0]) <= set("-: "):
                    rows[cells[0]] = dict(zip(head[1:], cells[1:]))
    except OSError:
        return {}, None
    return rows, os.path.relpath(path, ROOT)


def _profiled_traffic(kernel: str, stem: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    of this workload (calibrated against a plain copy kernel), or (None, None)."""
    rows, src = _profile_table(f"{stem}_hbm_traffic.md")
    try:
        r = rows[kernel]
        return (float(r["read GB"]) + float(r["write GB"])) * 1e9, src
    except (KeyError, ValueError):
        return None, None


def _profiled_valu(kernel: str, stem: str):
    """VALU and SALU wave instructions per launch of `kernel` from the committed rocprofv3 SQ
    counter summary of this workload, or (None, None, None)."""
    rows, src = _profile_table(f"{stem}_sq_counters.md")
    try:
        r = rows[kernel]
        return float(r["INSTS_VALU"]), float(r["INSTS_SALU"]), src
    except (KeyError, ValueError):
        return None, None, None


def _profiled_waves(kernel: str, stem: str):
    """Waves per launch of `kernel` in the committed SQ counter summary (one wave per vector for
    the beam layers), or None."""
    rows, _ = _profile_table(f"{stem}_sq_counters.md")
    try:
        return float(rows[kernel]["WAVES"])
    except (KeyError, ValueError):
        return None


def _roofline_valu(kernel: str, valu, avg_ms, src, per: str = "launch"):
    """The VALU-issue roofline of `kernel`: its SQ_INSTS_VALU per launch (committed profile of the
    same workload; `per` = "chunk" when both figures are summed over a streamed chunk's launches)
    over this run's average time for the same unit, against PEAK_VALU_WAVE_INSTS."""
    rate = valu / (avg_ms * 1e-3) if valu and avg_ms > 0 else None
    return {"kernel": kernel, "bound": "valu", "achieved": rate, "peak": PEAK_VALU_WAVE_INSTS,
            "unit": "wave-instructions/s", "frac": rate / PEAK_VALU_WAVE_INSTS if rate else None,
            f"valu_wave_insts_per_{per}": valu, ("avg_launch_ms" if per == "launch" else f"ms_per_{per}"): avg_ms,
            "valu_source": src}


def _calib_copy(ctx, mb: int):
    """A plain device copy of mb MiB (DevCopyKernel) whose FETCH_SIZE/WRITE_SIZE readings scale the
    counters of the profiled kernels to bytes."""
    if mb <= 0:
        return
    nb = mb * (1 << 20)
    a_ = ctx.dev_alloc(nb)
    b_ = ctx.dev_alloc(nb)
    ctx.lib.stlq_mi355_dev_copy_kernel(ctx.h, a_, b_, nb)
    ctx.synchronize()
    ctx.dev_free(a_)
    ctx.dev_free(b_)
    log(f"calibration copy of {mb} MiB done")


def _layer_kernel_name(L: int, lr: bool, last: bool = False) -> str:
    """The profiled name of the beam layer kernel that runs layer L with a full codebook in the
    best-first pass (the dispatch of LaunchL in beam_kernels.hpp): the survivor-queue kernel for layers
    1..8, then the staged kernel, for the full-precomp and the large-root beam alike; the
    last layer runs the kernel built for the final pick only (template flag LAST)."""
    tail = ", true" if last else ""
    kind = "LayerKernel" if L <= 8 else "LayerKernelStaged"
    return f"{kind}<{L}, {'true' if lr else 'false'}, true, true{tail}>"


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--n", type=int, default=0, help="vectors (0 = the configuration's size)")
    ap.add_argument("--cpu-sample", type=int, default=100_000,
                    help="vectors timed on the CPU oracle (0 = skip)")
    ap.add_argument("--config", default="C2", choices=["C1", "C2", "C3", "C4", "C5"],
                    help="benchmark configuration; C2 is the headline, the others are extra measurements")
    ap.add_argument("--chunk", type=int, default=4_000_000, help="C5 streaming chunk (vectors)")
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

    w = workloads.CONFIGS[args.config]
    if args.config == "C5":
        return bench_stream_large_root(args, w)
    n = int(args.n) or w.n
    t0 = time.perf_counter()
    mix = workloads.Mixture(w.kind, w.d, w.n_comp, w.seed)
    X = mix.sample(0, n)
    C = workloads.make_codebooks(w)
    h = [w.K] * w.m
    log(f"workload {w.name} generated in {time.perf_counter() - t0:.1f}s: n={n} d={w.d} M={w.m} K={w.K} "
        f"beam={w.H_beam} icm={w.icm_iters}")

    ctx = Context(0)
    dev_name, cus = ctx.device_info()
    ctx.set_codebooks(C, h)
    cfg = EncodeConfig(H_beam=w.H_beam, icm_iters=w.icm_iters, want_coeffs=True)
    dX = ctx.dev_alloc(X.nbytes)
    dcodes = ctx.dev_alloc(n * w.m)
    da = ctx.dev_alloc(n * w.m * 4)
    dcost = ctx.dev_alloc(n * 4)
    ctx.h2d(dX, X)

    for k in range(args.warmup):
        ctx.encode_device(dX, n, cfg, dcodes, da, dcost)
        ctx.synchronize()
        log(f"warmup step {k + 1}/{args.warmup} done")

    gemm_ms = beam_ms = total_ms = icm_ms = 0.0
    layer_ms = np.zeros(20)
    launches = reruns = 0
    ctx.synchronize()
    t_start = time.perf_counter()
    for k in range(args.steps):
        ctx.encode_device(dX, n, cfg, dcodes, da, dcost)
        t = ctx.last_timings()  # waits for this step's events
        gemm_ms += t.gemm_ms
        beam_ms += t.beam_ms
        icm_ms += t.icm_ms
        total_ms += t.total_ms
        layer_ms += np.array(t.layer_ms[:20])
        launches += t.gemm_launches
        reruns += t.beam_reruns
    ctx.synchronize()
    wall = time.perf_counter() - t_start
    log(f"timed {args.steps} steps in {wall:.3f}s")

    codes = ctx.d2h(np.empty((n, w.m), np.uint8), dcodes)
    cost = ctx.d2h(np.empty(n, np.float32), dcost)

    _calib_copy(ctx, args.calib_copy_mb)

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
        # vectors the best-first beam pass flagged and re-ran in the reference order (per step)
        "beam_reruns": reruns / steps,
        "icm_ms": icm_ms / steps,
        "device_total_ms": total_ms / steps,
    }

    # the timed layer kernel: full codebook, best-first pass (the default beam order)
    prof_kernel = _layer_kernel_name(last, lr=False, last=True)
    stem = f"{args.config.lower()}_encode"
    traffic, traffic_src = _profiled_traffic(prof_kernel, stem)
    valu, salu, valu_src = _profiled_valu(prof_kernel, stem)
    metric = ("vectors encoded/sec (d=128,M=8,K=256,B=16)" if args.config == "C2" else
              f"vectors encoded/sec (d={d},M={M},K={K},B={B}" + (f",ICM={w.icm_iters})" if w.icm_iters else ")"))
    workload = {
        "C1": "100k vectors d=128 (1024-component GMM, centres N(0,1), sigma 0.3), M=4 x K=256, beam 4",
        "C2": "1M descriptor-like vectors d=128 (4096-component GMM, clipped/rounded to [0,255], fp32), "
              "M=8 x K=256 residual k-means codebooks, beam 16, no ICM, LS refit + cost",
        "C3": "1M unit-norm vectors d=96 (8192-component spherical mixture, 0.2 rad), spherical k-means "
              "M=8 x K=256, beam 16 + 2 ICM sweeps (|score|), LS refit + cost",
        "C4": "500k vectors d=960 (2048 components, per-dim variance 1/(1+i/64)), M=16 x K=256, beam 8, "
              "LS refit + cost",
    }[args.config]
    out = {
        "metric": metric,
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
        "config": {"workload": workload, "name": args.config, "n": n, "d": d, "M": M, "K": K, "H_beam": B,
                   "icm_iters": w.icm_iters},
        "roofline": {
            "kernel": f"beam layer L={last} (LayerKernel<{last}>)",
            "bound": "hbm",
            "achieved": beam_ach,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": beam_ach / PEAK_HBM_GBS,
            "traffic": traffic,
            "traffic_source": traffic_src,
            "algorithmic_bytes_per_launch": sel_bytes,
            "avg_launch_ms": avg_last_ms,
        },
        # What bounds this kernel instead: VALU issue (the pruning test, the exact fp32 candidate
        # arithmetic of the survivors and the top-H replay).
        "roofline_valu": dict(_roofline_valu(prof_kernel, valu, avg_last_ms, valu_src),
                              salu_wave_insts_per_launch=salu),
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
        from oracle import ref

        ns = min(args.cpu_sample, n)
        threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
        use_ref = ref.available()
        Xs = X[:ns]
        G, inv = orc.build_precomp(C, h, nthreads=threads)
        tc = time.perf_counter()
        nx2 = ref.xnorm2(Xs) if use_ref else orc.xnorm2(Xs, nthreads=threads)
        xC = orc.gemm_xc(C, Xs, mode=1, nthreads=threads)
        t_gemm = time.perf_counter() - tc
        if use_ref:
            codes_o = ref.beam_search(Xs, xC, G, h, B)
        else:
            codes_o, _ = orc.beam_search(nx2, xC, G, h, B, nthreads=threads)
        t_beam = time.perf_counter() - tc - t_gemm
        if use_ref:
            if w.icm_iters:
                codes_o, a_o, cost_o = ref.icm(Xs, xC, G, inv, h, codes_o, w.icm_iters, True, cfg.seed)
            else:
                a_o = ref.solve_ls_all(xC, G, h, codes_o)
                cost_o = ref.compute_costs(xC, G, h, codes_o, a_o, nx2)
        elif w.icm_iters:
            codes_o, a_o, cost_o, _ = orc.icm(xC, G, inv, h, nx2, codes_o, w.icm_iters, True, cfg.seed,
                                              nthreads=threads)
        else:
            a_o, _ = orc.solve_ls_all(xC, G, h, codes_o, nthreads=threads)
            cost_o = orc.compute_costs(xC, G, h, codes_o, a_o, nx2, nthreads=threads)
        t_cpu = time.perf_counter() - tc
        log(f"cpu {'reference' if use_ref else 'oracle'}: {ns} vectors in {t_cpu:.1f}s on {threads} threads")
        cpu_model = _cpu_model()
        if use_ref:
            tail = "DynamicIcmWithIlsAbsNoNormal (ICM)" if w.icm_iters else "SolveLeastSquaresAll + ComputeCosts"
            what = (f"reference ComputeXNorm2 + BeamSearchPrefixLS + {tail}, compiled from its own sources "
                    f"(g++ -O3 -fopenmp; LAPACK from the image's MKL, sequential layer); xC by the oracle's "
                    f"fused-order dot (the reference's BLAS is not in the image)")
        else:
            what = f"oracle port: ||x||^2 + xC + beam + {'ICM ' if w.icm_iters else ''}LS refit + cost"
        out["cpu_baseline"] = {
            "value": ns / t_cpu,
            "unit": "vectors/s",
            "cores": threads,
            "kind": "reference" if use_ref else "port",
            "sample": f"first {ns} vectors of the same workload; {what}; "
                      f"stages s: ||x||^2+xC {t_gemm:.2f}, beam {t_beam:.2f}, rest {t_cpu - t_gemm - t_beam:.2f}; "
                      f"cpu: {cpu_model}",
        }
        same = np.all(codes[:ns] == codes_o, axis=1)
        diff_idx = np.nonzero(~same)[0]
        max_rel_mse = 0.0
        if diff_idx.size:
            ma = orc.mse_fp64_refit(Xs[diff_idx], C, h, codes_o[diff_idx], nthreads=threads)
            mb = orc.mse_fp64_refit(Xs[diff_idx], C, h, codes[:ns][diff_idx], nthreads=threads)
            max_rel_mse = float(np.max(np.abs(ma - mb) / np.maximum(np.abs(ma), 1e-30)))
        cg = cost[:ns].astype(np.float64)
        co = cost_o.astype(np.float64)
        out["parity"] = {
            "sample": ns,
            "against": "reference" if use_ref else "oracle",
            "codes_identical_frac": float(np.mean(same)),
            "differing_max_rel_mse_fp64": max_rel_mse,
            "cost_bit_identical_frac": float(np.mean(cost[:ns].view(np.uint32) == cost_o.view(np.uint32))),
            # the fp32 cost ||x||^2 - 2 a.xC + a'Ga cancels, so its rounding scales with ||x||^2
            "cost_max_diff_over_xnorm2": float(np.max(np.abs(cg - co) / np.maximum(nx2.astype(np.float64), 1e-30))),
        }

    for p in (dX, dcodes, da, dcost):
        ctx.dev_free(p)
    ctx.close()
    print(json.dumps(out), flush=True)


def bench_stream_large_root(args, w):
    """C5: streaming encode of uint8-valued descriptor vectors in pinned chunks, nearest root of a
    65,536-codeword root codebook forced, then 16 residual codebooks x 256, beam 32, then the
    large-root LS refit and per-vector cost (the coefficients the streaming encode stores)."""
    from stlq_amd import workloads
    from stlq_amd.encoder import Context, EncodeConfig

    h0 = int(w.extra["h0"])
    chunk = int(args.chunk)
    n = int(args.n) or 2 * chunk
    chunk = min(chunk, n)
    t0 = time.perf_counter()
    mix = workloads.Mixture(w.kind, w.d, w.n_comp, w.seed)
    # Every vector of the stream is drawn from the mixture by its global id while the previous
    # chunk encodes (fill runs on the host between chunk launches); row blocks in parallel.
    gen = cf.ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1))
    C0, Cs = workloads.make_large_root(w, h0, w.m - 1)
    h = [h0] + [w.K] * (w.m - 1)
    log(f"workload C5 generated in {time.perf_counter() - t0:.1f}s: stream n={n} chunk={chunk} d={w.d} "
        f"h0={h0} small={w.m - 1}x{w.K} beam={w.H_beam}")
    ctx = Context(0)
    dev_name, cus = ctx.device_info()
    ctx.set_large_root(C0, Cs, h)
    cfg = EncodeConfig(H_beam=w.H_beam, icm_iters=0, want_coeffs=True)
    keep = min(2000, chunk)
    first_codes = {}

    def fill(first, count, out):
        mix.sample_into(first, out, gen)  # values are integers in [0, 255]: exact as uint8

    t_prog = [time.perf_counter(), 0]

    def sink(first, count, res):
        t_prog[1] += 1
        if time.perf_counter() - t_prog[0] > 20.0:
            log(f"stream progress: {first + count} vectors written ({t_prog[1]} chunks)")
            t_prog[0] = time.perf_counter()
        if first == 0:
            first_codes["cid"] = res["cluster_id"][:keep].copy()
            first_codes["Bs"] = res["B_small"][:keep].copy()
            first_codes["a"] = res["a"][:keep].copy()
            first_codes["cost"] = res["cost"][:keep].copy()

    warm = min(chunk, 100_000)
    ctx.encode_stream(warm, warm, cfg, fill, sink, input_u8=True, large_root=True, root_mode=1)
    log("warmup stream done")
    t_start = time.perf_counter()
    t_prog[0] = t_start
    st = ctx.encode_stream(n, chunk, cfg, fill, sink, input_u8=True, large_root=True, root_mode=1)
    wall = time.perf_counter() - t_start
    t = ctx.last_timings()
    log(f"streamed {n} vectors in {wall:.2f}s ({st.chunks} chunks)")
    _calib_copy(ctx, args.calib_copy_mb)
    M = w.m
    last = M - 1
    layer_ms = np.array(t.layer_ms[:20])
    nch = max(st.chunks, 1)
    avg_last_ms = layer_ms[last] / nch
    sel_bytes = 4.0 * w.K * w.H_beam * chunk
    beam_ach = sel_bytes / (avg_last_ms * 1e-3) / 1e9
    h2d_gbs = st.h2d_bytes / (st.h2d_ms * 1e-3) / 1e9 if st.h2d_ms > 0 else None
    dist_flops = 2.0 * w.d * (h0 + (M - 1) * w.K) * (n / nch)
    dist_ach = dist_flops / (t.gemm_ms / nch * 1e-3) / 1e12 if t.gemm_ms > 0 else None
    prof_kernel = _layer_kernel_name(last, lr=True, last=True)
    traffic, traffic_src = _profiled_traffic(prof_kernel, "c5_stream")
    valu, _, valu_src = _profiled_valu(prof_kernel, "c5_stream")
    # A chunk's layer runs as one launch per workspace tile, and the counter runs used smaller
    # chunks: scale the profiled per-launch figures by vectors (one wave per vector) to a chunk.
    pw = _profiled_waves(prof_kernel, "c5_stream")
    per_chunk = chunk / pw if pw else None
    traffic = traffic * per_chunk if traffic and per_chunk else None
    valu = valu * per_chunk if valu and per_chunk else None
    out = {
        "metric": "vectors encoded/sec (stream, d=128 uint8, forced nearest root h0=65536 + 16x256, B=32)",
        "value": n / wall,
        "unit": "vectors/s",
        "n_gpus": 1,
        "steps": 1,
        "warmup": 1,
        "ms_per_step": wall * 1000.0,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"streaming encode of {n} uint8-valued d=128 vectors (C2 generator) in {chunk}-vector "
                               "pinned chunks, double-buffered H2D; nearest of 65,536 root codewords forced, then "
                               "16 residual codebooks x 256, beam 32, then the large-root LS refit and cost",
                   "name": "C5", "n": n, "chunk": chunk, "d": w.d, "h0": h0, "M_small": M - 1, "K": w.K,
                   "H_beam": w.H_beam},
        "roofline": {
            "kernel": f"large-root beam layer L={last} ({prof_kernel})",
            "bound": "hbm",
            "achieved": beam_ach,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": beam_ach / PEAK_HBM_GBS,
            "traffic": traffic,
            "traffic_source": traffic_src,
            # per chunk: the sum over the chunk's tile launches (bytes, counters and time alike)
            "algorithmic_bytes_per_chunk": sel_bytes,
            "ms_per_chunk": avg_last_ms,
        },
        "roofline_valu": _roofline_valu(prof_kernel, valu, avg_last_ms, valu_src, per="chunk"),
        # The distance stage: the nearest-root GEMM over the 65,536 roots (2*d*h0 flops per vector,
        # first-minimum epilogue) and the xC GEMM over the 16 x 256 small codewords (2*d*Hs), both
        # fp32 MFMA, timed together by HIP events with the NaN fix-up and the root-dot gather.
        "roofline_distance": {
            "kernel": "NearestRootKernel + GemmXcKernel (fp32 MFMA, lookup form)",
            "bound": "mfma",
            "achieved": dist_ach,
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": dist_ach / PEAK_FP32_MFMA_TFLOPS if dist_ach else None,
            "flops_per_chunk": dist_flops,
            "ms_per_chunk": t.gemm_ms / nch,
        },
        "streaming": {
            "h2d_GBps": h2d_gbs,
            "h2d_bytes": st.h2d_bytes,
            "h2d_ms": st.h2d_ms,
            "compute_ms": st.compute_ms,
            "fill_ms": st.fill_ms,
            "sink_ms": st.sink_ms,
            "wall_ms": st.wall_ms,
            "gpu_busy_frac": st.compute_ms / st.wall_ms if st.wall_ms > 0 else None,
        },
        "stages": {
            "gemm_ms_per_chunk": t.gemm_ms / nch,
            "root_seed_ms_per_chunk": layer_ms[0] / nch,
            "beam_layer_ms_per_chunk": [round(x / nch, 3) for x in layer_ms[:M]],
            "refit_ms_per_chunk": (t.ls_ms + t.icm_ms) / nch,
            "device_total_ms_per_chunk": t.total_ms / nch,
        },
        "device": {"arch": dev_name, "cus": cus},
    }
    if args.cpu_sample > 0:
        from oracle import oracle as orc
        from oracle import ref

        ns = min(args.cpu_sample, keep)
        threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
        use_ref = ref.available()
        Xs = mix.sample(0, min(chunk, 65536))[:ns]  # the stream's first rows (same row blocks)
        norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs, nthreads=threads)
        tc = time.perf_counter()
        nx2 = ref.xnorm2(Xs) if use_ref else orc.xnorm2(Xs, nthreads=threads)
        xs = orc.gemm_xc(Cs, Xs, mode=1, nthreads=threads)
        if use_ref:
            errs, rcodes, a0, r00 = orc.large_root_candidates(Xs, nx2, C0, norm0, w.H_beam, root_mode=1,
                                                              nthreads=threads)
            t_root = time.perf_counter() - tc
            cid_o, Bs_o = ref.expand_large_root(Gs, G0S, h, xs, w.H_beam, errs, rcodes, a0, r00)
            t_beam = time.perf_counter() - tc
            a_o = ref.solve_ls_all_large_root(Xs, C0, norm0, Gs, G0S, h, xs, cid_o, Bs_o)
            c_o = ref.compute_costs_large_root(Xs, C0, norm0, Gs, G0S, h, xs, cid_o, Bs_o, a_o, nx2)
        else:
            cid_o, Bs_o, _ = orc.beam_search_large_root(Xs, nx2, C0, norm0, xs, Gs, G0S, h, w.H_beam, root_mode=1,
                                                        nthreads=threads)
            t_root = 0.0
            t_beam = time.perf_counter() - tc
            a_o, _ = orc.solve_ls_all_large_root(Xs, C0, norm0, xs, Gs, G0S, h, cid_o, Bs_o, nthreads=threads)
            c_o = orc.compute_costs_large_root(Xs, C0, norm0, xs, Gs, G0S, h, cid_o, Bs_o, a_o, nx2, nthreads=threads)
        t_cpu = time.perf_counter() - tc
        log(f"cpu {'reference' if use_ref else 'oracle'}: {ns} vectors in {t_cpu:.1f}s on {threads} threads")
        if use_ref:
            what = (f"reference ComputeXNorm2 + BeamSearchPrefixLSLargeRootExpandFromRootCandidates + "
                    f"SolveLeastSquaresAllLargeRoot + ComputeCostsLargeRoot (its own sources, g++ -O3 -fopenmp, "
                    f"LAPACK from MKL for m=17) for the 16-layer beam 32 and the refit; xC_small and the "
                    f"nearest-root scan over 65,536 roots by the oracle (the reference's root GEMM needs BLAS); "
                    f"stages s: xnorm+xC+root {t_root:.2f}, expansion {t_beam - t_root:.2f}, refit "
                    f"{t_cpu - t_beam:.2f}")
        else:
            what = ("oracle port: ||x||^2 + xC_small + nearest-root scan over 65,536 roots + 16-layer beam 32 + "
                    "large-root LS refit and cost")
        out["cpu_baseline"] = {
            "value": ns / t_cpu, "unit": "vectors/s", "cores": threads,
            "kind": "reference" if use_ref else "port",
            "sample": f"first {ns} vectors of the stream; {what}; cpu: {_cpu_model()}"}
        same = (cid_o == first_codes["cid"][:ns]) & np.all(Bs_o == first_codes["Bs"][:ns], axis=1)
        cg = first_codes["cost"][:ns]
        rel = np.abs(cg[same].astype(np.float64) - c_o[same]) / np.maximum(nx2[same].astype(np.float64), 1e-30)
        out["parity"] = {"sample": ns, "against": "reference" if use_ref else "oracle",
                         "codes_identical_frac": float(np.mean(same)),
                         "costs_identical_frac": float(np.mean(cg[same].view(np.uint32) == c_o[same].view(np.uint32))),
                         "cost_max_rel_diff_vs_norm2": float(rel.max()) if rel.size else 0.0}
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
