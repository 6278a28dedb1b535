#!/usr/bin/env python3
"""Benchmark of the gfx950 GEMM engine on one MI355X.

Headline (the `value` of the JSON line): int8 GEMM i8 x i8 -> i32 at
M = N = K = 4096, A row-major, B column-major (transposed via strides), C
row-major, alpha = 1, beta = 0, inputs uniform over [-128, 127] from a seeded
xorshift* stream, resident in HBM before timing.  A "step" is one gemm_i8 call
through the C ABI (stream-ordered, no host sync inside the timed region).

The other workloads of the path are measured after it and reported under
"workloads" in the same line: the requantizing int8 linear layer with a
prepacked weight (2048 x 4096 x 11008, 16 calls), batched bf16 attention scores
(64 x 512 x 512 x 128, f32 out), bf16 4096^3 (the matrix-core-bound bf16
shape), int8 GEMV (W 14336 x 4096, M = 1 and 8; five weight copies rotate so
the 256 MB Infinity Cache cannot serve them), f32 GEMV 16384^2, and the f32
512^3 plumbing case.

roofline: algorithmic ops of one 4096^3 launch (2*4096^3) over the average
launch time measured with HIP events on the launch stream, against the
MI355X dense int8 peak (5.0 POP/s).  traffic: HBM bytes per launch from the
committed rocprofv3 counter summary (profiles/traffic.json), or null.
cpu_baseline: the oracle's C restatement of gemmkit's CPU i8 path (BLIS
5-loop + AVX-512 VNNI microkernel, OpenMP threads) on the host cores, 4096^3.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"int8": 5.0e15, "bf16": 2.5e15, "f32": 157.3e12, "hbm": 8.0e12}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra", action="store_true", help="headline workload only")
    p.add_argument("--only", default=None, help="run one workload by name (profiling)")
    return p.parse_args()


def timed(fn, steps, warmup, stream):
    """Average ms per call of `fn` over `steps` back-to-back calls, HIP events on
    the launch stream, synchronized on both sides."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the workload would shard by output tiles, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import gemmkit_amd as gk
    import oracle

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    gk.set_synchronous(False)
    props = torch.cuda.get_device_properties(0)
    workloads = {}

    def want(name):
        return args.only is None or args.only == name

    # ---------------------------------------------------------------- headline
    M = N = K = 4096
    a = oracle.rng_i8_full(1, M * K)
    b = oracle.rng_i8_full(2, K * N)
    ad = torch.from_numpy(a).to(dev)
    bd = torch.from_numpy(b).to(dev)
    cd = torch.empty(M * N, dtype=torch.int32, device=dev)
    av = gk.MatRef.from_row_major(ad, M, K)
    bv = gk.MatRef(bd, K, N, 1, K)
    cv = gk.MatMut.from_row_major(cd, M, N)
    i8_ms = None
    if want("i8_gemm_4096"):
        i8_ms = timed(lambda: gk.gemm_i8(1, av, bv, 0, cv), args.steps, args.warmup, stream)
        # spot check the timed output: row 17 against the oracle
        ref = np.zeros(N, np.int32)
        oracle.gemm_i8(1, K, N, 1, a[17 * K:18 * K], K, 1, b, 1, K, 0, ref, N, 1)
        ok = bool(np.array_equal(cd[17 * N:18 * N].cpu().numpy(), ref))
        workloads["i8_gemm_4096"] = {"ms": i8_ms, "TOPS": 2 * M * N * K / i8_ms / 1e9,
                                     "parity_row_check": ok}
    del cd

    # ------------------------------------------------------------------ extras
    if not args.no_extra:
        run_extras(args, workloads, want, dev, stream, gk, oracle, np, torch)

    # ------------------------------------------------------------ CPU baseline
    cpu = None
    if not args.no_cpu_baseline and args.only is None:
        cpu = cpu_baseline(oracle, np, a, b, M, N, K)

    ops = 2 * M * N * K
    value = ops / (i8_ms * 1e-3) / 1e12 if i8_ms else None
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("i8_gemm_4096", {}).get("hbm_bytes_per_launch")
    line = {
        "metric": "int8 GEMM TOPS + MFMA util at 4096³; bf16 TFLOPS; GEMV HBM GB/s",
        "value": value,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": i8_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded xorshift*, uniform i8 in [-128,127])",
        "config": {"workload": "gemm_i8 M=N=K=4096, A row-major, B col-major via strides, "
                               "C row-major i32, alpha=1, beta=0",
                   "device": props.name, "cus": props.multi_processor_count},
        "roofline": {"bound": "mfma", "achieved": value, "peak": PEAK["int8"] / 1e12,
                     "unit": "TOPS", "frac": (value * 1e12 / PEAK["int8"]) if value else None,
                     "traffic": traffic},
        "cpu_baseline": cpu,
        "workloads": workloads,
    }
    print(json.dumps(line))


def run_extras(args, workloads, want, dev, stream, gk, oracle, np, torch):
    steps = max(5, args.steps // 2)
    warm = max(2, args.warmup // 2)

    # int8 linear layer + requant, W prepacked once, 16 calls per step
    if want("i8_layer_requant"):
        T, K, Nc = 2048, 4096, 11008
        x = torch.from_numpy(oracle.rng_i8_sym127(21, T * K)).to(dev)
        w = torch.from_numpy(oracle.rng_i8_sym127(22, Nc * K)).to(dev)
        u = oracle.rng_unit(23, 2 * Nc)
        bias = torch.from_numpy(np.round(u[:Nc] * 65536).astype(np.int32)).to(dev)
        scale = torch.from_numpy((1e-4 + (u[Nc:] + 1) / 2 * (1e-2 - 1e-4)).astype(np.float32)).to(dev)
        # W as the prepacked B: B = W^T (K x Nc), element (p, j) at w[j*K + p]
        packed = gk.prepack_rhs_i8(gk.MatRef(w, K, Nc, 1, K))
        y = torch.empty(T * Nc, dtype=torch.int8, device=dev)
        req = gk.Requantize(gk.RequantScale.PerCol(scale), 0, bias, bias_axis="col", relu=True)
        xv = gk.MatRef.from_row_major(x, T, K)
        yv = gk.MatMut.from_row_major(y, T, Nc)

        def layer():
            for _ in range(16):
                gk.gemm_i8_packed_b_requant(xv, packed, req, yv)
        ms = timed(layer, max(2, steps // 8), 1, stream) / 16
        ops = 2 * T * K * Nc
        workloads["i8_layer_requant"] = {"ms_per_call": ms, "TOPS": ops / ms / 1e9,
                                         "frac_int8_peak": ops / (ms * 1e-3) / 5.0e15}
        del x, w, y, packed

    # batched bf16 attention scores, f32 out
    if want("bf16_batched_attn"):
        Bt, S, D = 64, 512, 128
        q = torch.randn(Bt * S * D, device=dev).to(torch.bfloat16)
        kk = torch.randn(Bt * S * D, device=dev).to(torch.bfloat16)
        out = torch.empty(Bt * S * S, dtype=torch.float32, device=dev)
        alpha = 1.0 / np.sqrt(128.0)
        fn = lambda: gk.gemm_batched_bf16_f32out(  # noqa: E731
            Bt, alpha, gk.MatRef.from_row_major(q, S, D), S * D, gk.MatRef(kk, D, S, 1, D), S * D,
            0.0, gk.MatMut.from_row_major(out, S, S), S * S)
        ms = timed(fn, steps, warm, stream)
        byts = 2 * Bt * S * D * 2 + Bt * S * S * 4
        workloads["bf16_batched_attn"] = {"ms": ms, "TFLOPS": 2 * Bt * S * S * D / ms / 1e9,
                                          "GBps": byts / ms / 1e6,
                                          "frac_hbm": byts / (ms * 1e-3) / 8.0e12}
        del q, kk, out

    # bf16 4096^3 (matrix-core bound), f32 out
    if want("bf16_gemm_4096"):
        n = 4096
        a = torch.randn(n * n, device=dev).to(torch.bfloat16)
        b = torch.randn(n * n, device=dev).to(torch.bfloat16)
        c = torch.empty(n * n, dtype=torch.float32, device=dev)
        fn = lambda: gk.gemm_bf16_f32out(1.0, gk.MatRef.from_row_major(a, n, n),  # noqa: E731
                                         gk.MatRef(b, n, n, 1, n), 0.0,
                                         gk.MatMut.from_row_major(c, n, n))
        ms = timed(fn, steps, warm, stream)
        workloads["bf16_gemm_4096"] = {"ms": ms, "TFLOPS": 2 * n ** 3 / ms / 1e9,
                                       "frac_bf16_peak": 2 * n ** 3 / (ms * 1e-3) / 2.5e15}
        del a, b, c

    # int8 GEMV, W 14336 x 4096, M = 1 and 8; five weight copies rotate
    if want("i8_gemv"):
        Nw, K = 14336, 4096
        copies = [torch.from_numpy(oracle.rng_i8_sym127(31 + i, Nw * K)).to(dev) for i in range(5)]
        for Mv in (1, 8):
            x = torch.from_numpy(oracle.rng_i8_sym127(40 + Mv, Mv * K)).to(dev)
            y = torch.empty(Mv * Nw, dtype=torch.int32, device=dev)
            state = {"i": 0}

            def fn():
                w = copies[state["i"] % 5]
                state["i"] += 1
                gk.gemm_i8(1, gk.MatRef.from_row_major(x, Mv, K), gk.MatRef(w, K, Nw, 1, K), 0,
                           gk.MatMut.from_row_major(y, Mv, Nw))
            ms = timed(fn, steps * 2, warm, stream)
            byts = Nw * K + Mv * K + Mv * Nw * 4
            workloads[f"i8_gemv_m{Mv}"] = {"ms": ms, "GBps": byts / ms / 1e6,
                                           "frac_hbm": byts / (ms * 1e-3) / 8.0e12}
        del copies

    # f32 GEMV 16384^2 (1 GiB matrix, larger than the Infinity Cache)
    if want("f32_gemv"):
        n = 16384
        A = torch.randn(n * n, device=dev)
        xv = torch.randn(n, device=dev)
        yv = torch.empty(n, device=dev)
        fn = lambda: gk.gemm(1.0, gk.MatRef.from_row_major(A, n, n),  # noqa: E731
                             gk.MatRef(xv, n, 1, 1, 1), 0.0, gk.MatMut(yv, n, 1, 1, 1))
        ms = timed(fn, steps, warm, stream)
        byts = n * n * 4 + n * 4 + n * 4
        workloads["f32_gemv_16384"] = {"ms": ms, "GBps": byts / ms / 1e6,
                                       "frac_hbm": byts / (ms * 1e-3) / 8.0e12}
        del A

    # f32 512^3 plumbing (all row-major)
    if want("f32_gemm_512"):
        n = 512
        a = torch.rand(n * n, device=dev) * 2 - 1
        b = torch.rand(n * n, device=dev) * 2 - 1
        c = torch.empty(n * n, device=dev)
        fn = lambda: gk.gemm(1.0, gk.MatRef.from_row_major(a, n, n),  # noqa: E731
                             gk.MatRef.from_row_major(b, n, n), 0.0,
                             gk.MatMut.from_row_major(c, n, n))
        ms = timed(fn, steps, warm, stream)
        workloads["f32_gemm_512"] = {"ms": ms, "TFLOPS": 2 * n ** 3 / ms / 1e9}


def cpu_baseline(oracle, np, a, b, M, N, K):
    """gemmkit's CPU i8 path restated in C (oracle/cpu_port.c), timed as the
    reference's perf harness does: 3 warmups, batches calibrated to ~70 ms,
    median of 9 (tests/perf/harness.rs:32-120).  Bounded to ~10-20 s."""
    c = np.empty(M * N, np.int32)
    threads = oracle.port_max_threads()
    run = lambda: oracle.port_gemm_i8(M, K, N, 1, a, K, 1, b, 1, K, 0, c, N, 1, threads)  # noqa: E731
    for _ in range(3):
        run()
    t0 = time.perf_counter()
    run()
    one = time.perf_counter() - t0
    iters = max(1, int(0.07 / max(one, 1e-6)))
    rates = []
    deadline = time.perf_counter() + 20.0
    for _ in range(9):
        t0 = time.perf_counter()
        for _ in range(iters):
            run()
        dt = (time.perf_counter() - t0) / iters
        rates.append(2 * M * N * K / dt / 1e12)
        if time.perf_counter() > deadline:
            break
    rates.sort()
    return {"value": rates[len(rates) // 2], "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"full 4096^3 gemm_i8 (A row-major, B col-major), {len(rates)} batches of "
                      f"{iters}; median; min {rates[0]:.3f} max {rates[-1]:.3f}; "
                      f"AVX-512 VNNI={'yes' if oracle.port_has_vnni() else 'no'}"}


if __name__ == "__main__":
    main()
