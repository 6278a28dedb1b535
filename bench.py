#!/usr/bin/env python3
"""Benchmark of the gfx950 GEMM engine on one MI355X.

Headline (the `value` of the JSON line): int8 GEMM i8 x i8 -> i32 at
M = N = K = 4096, A row-major, B column-major (transposed via strides), C
row-major, alpha = 1, beta = 0, inputs uniform over [-128, 127] from a seeded
xorshift* stream, resident in HBM before timing.  A "step" is one gemm_i8 call
through the C ABI.  The K calls are timed two ways on the launch stream:
issued back to back from the host (eager, stream-ordered, the host running
ahead of the device), and as a HIP graph of the same C-ABI calls, replayed
(no host overhead at all).  HIP events on that stream bracket each of 7
repetitions, with a device synchronize on both sides; the reported time is the
faster way's median (min and max beside it, as the reference's harness reports
them, tests/perf/harness.rs:62-120), and both ways' medians are in the line
(ms_eager, ms_graph, launch).  On this ROCm the graph's kernel nodes run
6-12% longer than the same kernels launched eagerly, so the long kernels time
faster eager and the short, launch-bound ones faster as a graph.  Before that,
untimed warmup calls run for at least --warmup calls and --warmup-ms of wall
time (300 ms by default): from idle the GPU takes some 100 ms of load to raise
its clocks, and a shorter warmup times the ramp instead of the steady state.

The other workloads of the path follow under "workloads", each with its own
roofline (achieved rate against the bound that limits it) and CPU baseline:
the requantizing int8 linear layer with a prepacked weight (2048 x 4096 x
11008, 16 calls per step), batched bf16 attention scores (64 x 512 x 512 x 128,
f32 out; five input/output sets rotate so the 256 MB Infinity Cache cannot
serve them), bf16 4096^3 (the matrix-core-bound bf16 shape), int8 GEMV (W
14336 x 4096, M = 1 and 8; five weight copies rotate), f32 GEMV 16384^2, the f32
512^3 case, bf16 4096^3 with a fused bias and ReLU, and prepacked weights at
small batch (k = n = 2048, m = 8 and 64).

roofline: algorithmic work of one launch (ops, or bytes for the HBM-bound
shapes) over the median launch time from the HIP events, against MI355X's
published peaks (int8 5.0 POP/s, bf16 2.5 PFLOP/s, f32 matrix 157.3 TFLOP/s,
HBM 8 TB/s).  traffic: HBM bytes per call from the committed rocprofv3
counter summary (profiles/traffic.json), or null.
mfma_util: the headline kernel's matrix-core utilisation from the committed
rocprofv3 counter summary (profiles/mfma_util.json), or null.
cpu_baseline: the oracle's C restatement of gemmkit's CPU paths
(oracle/cpu_port.c: BLIS 5-loop with the AVX-512 VNNI / FMA / BF16-dot
microtiles, the dot_rows GEMV; OpenMP threads) on the host cores, Serial and
all cores, timed the way gemmkit's perf harness times (3 warmups, batches
calibrated to ~70 ms, median of up to 9), each leg bounded to a few seconds;
where a Serial run of the whole workload would take longer, a stated sample
of it is timed and the rate is over that sample's work.
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
ROTATE = 5  # input/output sets cycled through for the HBM-bound workloads


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--warmup-ms", type=float, default=300.0,
                   help="keep issuing untimed warmup calls until this much time has passed "
                        "(the GPU raises its clocks only after some 100 ms of load)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra", action="store_true", help="headline workload only")
    p.add_argument("--only", default=None, help="run one workload by name (profiling)")
    p.add_argument("--eager", action="store_true", help="time eager calls only (no graph)")
    p.add_argument("--graph", action="store_true", help="time graph replays only (no eager)")
    return p.parse_args()


class Timer:
    """Times `steps` calls of `fn` (a list of callables cycled in order) on the
    current stream, two ways: eager (the calls issued back to back from the
    host, stream-ordered) and as a HIP graph holding the same calls, replayed;
    each way `replays` times, each bracketed by HIP events on that stream with
    a device synchronize on both sides.  Returns the per-call time of the
    faster way (the median over its replays); `last` keeps that way's min and
    max (the reference's harness reports the median with its spread,
    tests/perf/harness.rs:62-120) and both ways' medians.  Long kernels run
    faster eager: the graph's kernel nodes take 6-12% longer each (int8
    4096^3: 63-65 against 57-58 us per call, the kernel's own duration in
    the trace 65.9 against 56.4 us), while short launch-bound ones gain from
    the graph.  mode "eager" or "graph" times one way only."""

    def __init__(self, mode: str, warmup_ms: float, replays: int = 7):
        self.mode = mode
        self.warmup_ms = warmup_ms
        self.replays = max(1, replays)
        self.last = {}

    def _eager(self, fns, steps, stream, start, stop):
        import torch
        times = []
        for _ in range(self.replays):
            start.record(stream)
            for i in range(steps):
                fns[i % len(fns)]()
            stop.record(stream)
            torch.cuda.synchronize()
            times.append(start.elapsed_time(stop) / steps)
        return sorted(times)

    def _graph(self, fns, steps, stream, start, stop):
        import torch
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for i in range(steps):
                    fns[i % len(fns)]()
        stream.wait_stream(side)
        graph.replay()  # untimed replay: first-launch costs
        torch.cuda.synchronize()
        times = []
        for _ in range(self.replays):
            start.record(stream)
            graph.replay()
            stop.record(stream)
            torch.cuda.synchronize()
            times.append(start.elapsed_time(stop) / steps)
        del graph
        return sorted(times)

    def __call__(self, fns, steps: int, warmup: int) -> float:
        import torch
        if callable(fns):
            fns = [fns]
        # Untimed warmup: at least `warmup` calls, and at least warmup_ms of
        # wall time with the device kept busy (synchronizing every 32 calls
        # so the host does not run ahead of it).
        t0 = time.perf_counter()
        i = 0
        while i < max(warmup, len(fns)) or (time.perf_counter() - t0) * 1e3 < self.warmup_ms:
            fns[i % len(fns)]()
            i += 1
            if i % 32 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        ways = {}
        if self.mode in ("both", "eager"):
            ways["eager"] = self._eager(fns, steps, stream, start, stop)
        if self.mode in ("both", "graph"):
            ways["graph"] = self._graph(fns, steps, stream, start, stop)
        best = min(ways, key=lambda w: ways[w][len(ways[w]) // 2])
        times = ways[best]
        med = times[len(times) // 2]
        self.last = {"ms_min": times[0], "ms_max": times[-1], "replays": len(times),
                     "launch": best}
        for w, t in ways.items():
            self.last[f"ms_{w}"] = t[len(t) // 2]
        return med


def roofline(bound: str, work: float, ms: float, traffic=None) -> dict:
    """Achieved rate of `work` (ops, or bytes for bound "hbm") in `ms` against
    the published peak of `bound` ("int8", "bf16", "f32" matrix, "hbm")."""
    rate = work / (ms * 1e-3)
    if bound == "hbm":
        return {"bound": "hbm", "achieved": rate / 1e9, "peak": PEAK["hbm"] / 1e9, "unit": "GB/s",
                "frac": rate / PEAK["hbm"], "traffic": traffic}
    unit = "TOPS" if bound == "int8" else "TFLOP/s"
    return {"bound": "mfma", "dtype": bound, "achieved": rate / 1e12, "peak": PEAK[bound] / 1e12,
            "unit": unit, "frac": rate / PEAK[bound], "traffic": traffic}


def load_traffic():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


# ---------------------------------------------------------------- CPU baseline

def cpu_rate(run, work: float, budget_s: float, scale: float = 1e12):
    """gemmkit's perf harness (tests/perf/harness.rs:32-120): 3 warmups, then
    batches of calls calibrated to ~70 ms, the median rate of up to 9 batches
    with min and max, stopping early when `budget_s` has passed.  Returns
    (median, min, max, batches, calls per batch) in units of `scale`."""
    t_end = time.perf_counter() + budget_s
    t0 = time.perf_counter()
    run()
    one = time.perf_counter() - t0
    for _ in range(2):
        if time.perf_counter() + one > t_end:
            break
        run()
    iters = max(1, int(0.07 / max(one, 1e-6)))
    rates = []
    while len(rates) < 9:
        t0 = time.perf_counter()
        for _ in range(iters):
            run()
        dt = (time.perf_counter() - t0) / iters
        rates.append(work / dt / scale)
        if time.perf_counter() + dt * iters > t_end and len(rates) >= 3:
            break
    rates.sort()
    return rates[len(rates) // 2], rates[0], rates[-1], len(rates), iters


def cpu_legs(legs, unit: str, scale: float, oracle):
    """legs: {"serial": (run, work, budget_s, sample), "all_cores": ...}, each
    `run` a callable taking the thread count.  Returns the baseline object:
    all-cores figures at the top level (value/unit/cores/kind/sample) and the
    Serial leg under "serial"."""
    out = {}
    nt = oracle.port_max_threads()
    for name, (run, work, budget, sample) in legs.items():
        threads = 1 if name == "serial" else nt
        med, lo, hi, nb, it = cpu_rate(lambda: run(threads), work, budget, scale)
        out[name] = {"value": med, "unit": unit, "cores": threads, "kind": "port",
                     "sample": f"{sample}; {nb} batches of {it}; median; min {lo:.4g} "
                               f"max {hi:.4g}"}
    top = dict(out.get("all_cores", {}))
    if "serial" in out:
        top["serial"] = out["serial"]
    isa = (f"AVX-512F={'yes' if oracle.port_has_avx512f() else 'no'}, "
           f"VNNI={'yes' if oracle.port_has_vnni() else 'no'}, "
           f"BF16={'yes' if oracle.port_has_bf16() else 'no'}")
    top["host_isa"] = isa
    top["host_cpu"] = host_cpu()
    return top


def host_cpu() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the workloads would shard by output tiles across GPUs)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    import gemmkit_amd as gk

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gk.set_synchronous(False)
    timed = Timer("eager" if args.eager else ("graph" if args.graph else "both"), args.warmup_ms)
    props = torch.cuda.get_device_properties(0)
    workloads = {}
    traffic_all = load_traffic()
    cpu_on = not args.no_cpu_baseline and args.only is None
    oracle = None
    if cpu_on or args.only in (None, "i8_gemm_4096"):
        import oracle  # the checker and the CPU-baseline port (test infrastructure)

    def want(name):
        return args.only is None or args.only == name

    if oracle is not None:
        gen_a = oracle.rng_i8_full(1, 4096 * 4096)
        gen_b = oracle.rng_i8_full(2, 4096 * 4096)
    else:
        g = torch.Generator().manual_seed(1)
        gen_a = torch.randint(-128, 128, (4096 * 4096,), dtype=torch.int8, generator=g).numpy()
        gen_b = torch.randint(-128, 128, (4096 * 4096,), dtype=torch.int8, generator=g).numpy()

    # ---------------------------------------------------------------- headline
    M = N = K = 4096
    ops = 2 * M * N * K
    ad = torch.from_numpy(gen_a).to(dev)
    bd = torch.from_numpy(gen_b).to(dev)
    cd = torch.empty(M * N, dtype=torch.int32, device=dev)
    i8_ms = None
    if want("i8_gemm_4096"):
        call = lambda: gk.gemm_i8_unchecked(M, K, N, 1, ad, K, 1, bd, 1, K, 0, cd, N, 1)  # noqa: E731
        i8_ms = timed(call, args.steps, args.warmup)
        entry = {"ms": i8_ms, "TOPS": ops / i8_ms / 1e9, **timed.last}
        if oracle is not None:
            # spot check the timed output: row 17 against the oracle
            ref = np.zeros(N, np.int32)
            oracle.gemm_i8(1, K, N, 1, gen_a[17 * K:18 * K], K, 1, gen_b, 1, K, 0, ref, N, 1)
            entry["parity_row_check"] = bool(np.array_equal(cd[17 * N:18 * N].cpu().numpy(), ref))
        workloads["i8_gemm_4096"] = entry
    del cd

    # ------------------------------------------------------------------ extras
    if not args.no_extra:
        run_extras(args, workloads, want, timed, dev, gk, np, torch, traffic_all,
                   oracle if cpu_on else None)

    # ------------------------------------------------------------ CPU baseline
    cpu = None
    if cpu_on:
        c_host = np.empty(M * N, np.int32)
        rows_s = 512  # Serial: the first 512 rows of A against all of B

        def run_i8(threads, rows=M):
            oracle.port_gemm_i8(rows, K, N, 1, gen_a, K, 1, gen_b, 1, K, 0, c_host, N, 1, threads)

        cpu = cpu_legs({
            "all_cores": (run_i8, ops, 20.0,
                          "full 4096^3 gemm_i8 (A row-major, B col-major) on the same inputs"),
            "serial": (lambda t: run_i8(t, rows_s), 2 * rows_s * N * K, 10.0,
                       f"the first {rows_s} rows of A (1/8 of the work) against the full B"),
        }, "TOPS", 1e12, oracle)
        workloads.setdefault("i8_gemm_4096", {})["cpu_baseline"] = cpu

    value = ops / (i8_ms * 1e-3) / 1e12 if i8_ms else None
    traffic = traffic_all.get("i8_gemm_4096", {}).get("hbm_bytes_per_launch")
    mfma_util = None
    upath = os.path.join(ROOT, "profiles", "mfma_util.json")
    if os.path.exists(upath):
        with open(upath) as f:
            u = json.load(f).get("i8_gemm_4096")
        if u:
            # GRBM_GUI_ACTIVE does not tick at the shader clock (a shader-clock
            # counter, s_memtime against the 100 MHz s_memrealtime, puts the
            # shader clock of this kernel at about 1.75 GHz where the GRBM
            # figure reads above 2.1), so the rate it gives is reported under
            # its own name.
            mfma_util = {"value": u["mfma_util"], "grbm_gui_active_ghz": u["clock_ghz"],
                         "source": "rocprofv3 SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD "
                                   "x 1024 SIMDs) (rocprof's MfmaUtil), eager launches; "
                                   "profiles/mfma_util.json"}
    line = {
        "metric": "int8 GEMM TOPS + MFMA util at 4096³; bf16 TFLOPS; GEMV HBM GB/s",
        "value": value,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_ms_min": args.warmup_ms,
        "ms_per_step": i8_ms,
        # spread of the per-call time over the timed replays (median above)
        "ms_min": workloads.get("i8_gemm_4096", {}).get("ms_min"),
        "ms_max": workloads.get("i8_gemm_4096", {}).get("ms_max"),
        "replays": workloads.get("i8_gemm_4096", {}).get("replays"),
        "launch": workloads.get("i8_gemm_4096", {}).get("launch"),
        "ms_eager": workloads.get("i8_gemm_4096", {}).get("ms_eager"),
        "ms_graph": workloads.get("i8_gemm_4096", {}).get("ms_graph"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded xorshift*, uniform i8 in [-128,127])",
        "config": {"workload": "gemm_i8 M=N=K=4096, A row-major, B col-major via strides, "
                               "C row-major i32, alpha=1, beta=0",
                   "device": props.name, "cus": props.multi_processor_count,
                   "timing": "the K calls back to back on one stream (eager) and as a replayed "
                             "HIP graph, 7 times each; the faster way's median (both in ms_eager "
                             "and ms_graph)"},
        "roofline": {"bound": "mfma", "achieved": value, "peak": PEAK["int8"] / 1e12,
                     "unit": "TOPS", "frac": (value * 1e12 / PEAK["int8"]) if value else None,
                     "traffic": traffic},
        "mfma_util": mfma_util,
        "cpu_baseline": cpu,
        "workloads": workloads,
    }
    print(json.dumps(line), flush=True)


def run_extras(args, workloads, want, timed, dev, gk, np, torch, traffic_all, oracle):
    """The other workloads of the path; `oracle` (the CPU port) is None when
    the CPU baselines are off."""
    steps = max(5, args.steps // 2)
    warm = max(2, args.warmup // 2)
    g = torch.Generator(device="cpu").manual_seed(7)

    def i8(n):
        return torch.randint(-127, 128, (n,), dtype=torch.int8, generator=g).to(dev)

    def tr(name):
        return traffic_all.get(name, {}).get("hbm_bytes_per_launch")

    def host(t):
        return np.ascontiguousarray(t.cpu().numpy())

    # int8 linear layer + requant, W prepacked once, 16 calls per step
    if want("i8_layer_requant"):
        T, K, Nc = 2048, 4096, 11008
        x, w = i8(T * K), i8(Nc * K)
        bias = torch.randint(-65536, 65537, (Nc,), dtype=torch.int32, generator=g).to(dev)
        scale = (1e-4 + torch.rand(Nc, generator=g) * (1e-2 - 1e-4)).to(dev)
        # W as the prepacked B: B = W^T (K x Nc), element (p, j) at w[j*K + p]
        packed = gk.prepack_rhs_i8(gk.MatRef(w, K, Nc, 1, K))
        y = torch.empty(T * Nc, dtype=torch.int8, device=dev)
        call = lambda: gk.gemm_i8_packed_b_requant_unchecked(  # noqa: E731
            T, x, K, 1, packed, 0.0, scale, 0, bias, y, Nc, 1, axis=1, relu=True)
        ms = timed(call, 16 * max(1, steps // 8), 2)
        ops = 2 * T * K * Nc
        e = {"ms_per_call": ms, "calls_per_step": 16, **timed.last, "TOPS": ops / ms / 1e9,
             "frac_int8_peak": ops / (ms * 1e-3) / PEAK["int8"],
             "roofline": roofline("int8", ops, ms, tr("i8_layer_requant"))}
        if oracle is not None:
            xh, wh, bh, sh = host(x), host(w), host(bias), host(scale)
            yh = np.empty(T * Nc, np.uint8)
            pb = oracle.PortPackedB(K, Nc, wh, 1, K)
            ts = 256  # Serial: 256 tokens

            def run(threads, tokens=T):
                oracle.port_gemm_i8_requant(tokens, K, Nc, xh, K, 1, None, 0, 0, 0.0, sh, 0, bh,
                                            1, 0, 127, yh, Nc, 1, threads, packed=pb)
            e["cpu_baseline"] = cpu_legs({
                "all_cores": (run, ops, 8.0, "the full layer per call (2048 tokens) on the same "
                                             "inputs, W prepacked once"),
                "serial": (lambda t: run(t, ts), 2 * ts * K * Nc, 6.0,
                           f"the first {ts} tokens (1/8 of a call) on the same prepacked W"),
            }, "TOPS", 1e12, oracle)
            del pb
        workloads["i8_layer_requant"] = e
        del x, w, y, packed

    # batched bf16 attention scores, f32 out; ROTATE sets cycle (84 MB each)
    if want("bf16_batched_attn"):
        Bt, S, D = 64, 512, 128
        sets = []
        for _ in range(ROTATE):
            q = torch.randn(Bt * S * D, generator=g).to(torch.bfloat16).to(dev)
            kk = torch.randn(Bt * S * D, generator=g).to(torch.bfloat16).to(dev)
            out = torch.empty(Bt * S * S, dtype=torch.float32, device=dev)
            sets.append((q, kk, out))
        alpha = 1.0 / np.sqrt(128.0)
        calls = [lambda q=q, kk=kk, out=out: gk.gemm_batched_bf16_f32out(
            Bt, alpha, gk.MatRef.from_row_major(q, S, D), S * D, gk.MatRef(kk, D, S, 1, D), S * D,
            0.0, gk.MatMut.from_row_major(out, S, S), S * S) for q, kk, out in sets]
        ms = timed(calls, 10 * len(calls), warm)
        byts = 2 * Bt * S * D * 2 + Bt * S * S * 4
        flops = 2 * Bt * S * S * D
        e = {"ms": ms, **timed.last, "sets_rotated": ROTATE, "TFLOPS": flops / ms / 1e9,
             "GBps": byts / ms / 1e6, "frac_hbm": byts / (ms * 1e-3) / PEAK["hbm"],
             "roofline": roofline("hbm", byts, ms, tr("bf16_batched_attn"))}
        if oracle is not None:
            qh = host(sets[0][0].view(torch.int16)).view(np.uint16)
            kh = host(sets[0][1].view(torch.int16)).view(np.uint16)
            oh = np.empty(Bt * S * S, np.float32)

            def run(threads):
                oracle.port_gemm_batched_bf16_f32out(Bt, S, D, S, alpha, qh, D, 1, S * D, kh, 1,
                                                     D, S * D, 0.0, oh, S, 1, S * S, threads)
            sample = "the full batch (64 x 512 x 512 x 128) on the first input set"
            e["cpu_baseline"] = cpu_legs({"all_cores": (run, flops, 6.0, sample),
                                          "serial": (run, flops, 6.0, sample)},
                                         "TFLOP/s", 1e12, oracle)
        workloads["bf16_batched_attn"] = e
        del sets

    # bf16 4096^3 (matrix-core bound), f32 out
    if want("bf16_gemm_4096"):
        n = 4096
        a = torch.randn(n * n, generator=g).to(torch.bfloat16).to(dev)
        b = torch.randn(n * n, generator=g).to(torch.bfloat16).to(dev)
        c = torch.empty(n * n, dtype=torch.float32, device=dev)
        call = lambda: gk.gemm_bf16_f32out(1.0, gk.MatRef.from_row_major(a, n, n),  # noqa: E731
                                           gk.MatRef(b, n, n, 1, n), 0.0,
                                           gk.MatMut.from_row_major(c, n, n))
        ms = timed(call, steps, warm)
        flops = 2 * n ** 3
        e = {"ms": ms, **timed.last, "TFLOPS": flops / ms / 1e9,
             "frac_bf16_peak": flops / (ms * 1e-3) / PEAK["bf16"],
             "roofline": roofline("bf16", flops, ms, tr("bf16_gemm_4096"))}
        if oracle is not None:
            ah = host(a.view(torch.int16)).view(np.uint16)
            bh = host(b.view(torch.int16)).view(np.uint16)
            ch = np.empty(n * n, np.float32)

            def run(threads, rows=n):
                oracle.port_gemm_batched_bf16_f32out(1, rows, n, n, 1.0, ah, n, 1, 0, bh, 1, n, 0,
                                                     0.0, ch, n, 1, 0, threads)
            rs = 256
            e["cpu_baseline"] = cpu_legs({
                "all_cores": (run, flops, 8.0, "full 4096^3 bf16 -> f32 on the same inputs"),
                "serial": (lambda t: run(t, rs), 2 * rs * n * n, 6.0,
                           f"the first {rs} rows of A (1/16 of the work) against the full B"),
            }, "TFLOP/s", 1e12, oracle)
        workloads["bf16_gemm_4096"] = e
        del a, b, c

    # int8 GEMV, W 14336 x 4096, M = 1 and 8; ROTATE weight copies
    if want("i8_gemv"):
        Nw, K = 14336, 4096
        copies = [i8(Nw * K) for _ in range(ROTATE)]
        for Mv in (1, 8):
            x = i8(Mv * K)
            y = torch.empty(Mv * Nw, dtype=torch.int32, device=dev)
            calls = [lambda w=w: gk.gemm_i8_unchecked(Mv, K, Nw, 1, x, K, 1, w, 1, K, 0, y, Nw, 1)
                     for w in copies]
            ms = timed(calls, 10 * len(calls), warm)
            byts = Nw * K + Mv * K + Mv * Nw * 4
            name = f"i8_gemv_m{Mv}"
            e = {"ms": ms, **timed.last, "GBps": byts / ms / 1e6,
                 "frac_hbm": byts / (ms * 1e-3) / PEAK["hbm"],
                 "roofline": roofline("hbm", byts, ms, tr(name))}
            if oracle is not None:
                xh, wh = host(x), host(copies[0])
                yh = np.empty(Mv * Nw, np.int32)

                def run(threads):
                    oracle.port_gemm_i8(Mv, K, Nw, 1, xh, K, 1, wh, 1, K, 0, yh, Nw, 1, threads)
                sample = (f"the full product (M = {Mv}) through the CPU i8 GEMM, which packs the "
                          "weight every call as the reference's gemm_i8 does")
                e["cpu_baseline"] = cpu_legs({"all_cores": (run, byts, 4.0, sample),
                                              "serial": (run, byts, 4.0, sample)},
                                             "GB/s", 1e9, oracle)
            workloads[name] = e
        del copies

    # f32 GEMV 16384^2 (1 GiB matrix, larger than the Infinity Cache)
    if want("f32_gemv"):
        n = 16384
        A = torch.randn(n * n, generator=g).to(dev)
        xv = torch.randn(n, generator=g).to(dev)
        yv = torch.empty(n, device=dev)
        call = lambda: gk.gemm_unchecked(n, n, 1, 1.0, A, n, 1, xv, 1, 1, 0.0, yv, 1, 1)  # noqa: E731
        ms = timed(call, steps, warm)
        byts = n * n * 4 + n * 4 + n * 4
        e = {"ms": ms, **timed.last, "GBps": byts / ms / 1e6,
             "frac_hbm": byts / (ms * 1e-3) / PEAK["hbm"],
             "roofline": roofline("hbm", byts, ms, tr("f32_gemv_16384"))}
        if oracle is not None:
            Ah, xh = host(A), host(xv)
            yh = np.empty(n, np.float32)

            def run(threads):
                oracle.port_gemv_f32(n, n, 1.0, Ah, n, xh, 0.0, yh, 1, threads)
            sample = "the full 16384^2 GEMV on the same inputs (dot_rows, rows across threads)"
            e["cpu_baseline"] = cpu_legs({"all_cores": (run, byts, 5.0, sample),
                                          "serial": (run, byts, 5.0, sample)},
                                         "GB/s", 1e9, oracle)
            del Ah
        workloads["f32_gemv_16384"] = e
        del A

    # f32 512^3 (all row-major; B goes through the pack into k-contiguous form)
    if want("f32_gemm_512"):
        n = 512
        a = (torch.rand(n * n, generator=g) * 2 - 1).to(dev)
        b = (torch.rand(n * n, generator=g) * 2 - 1).to(dev)
        c = torch.empty(n * n, device=dev)
        call = lambda: gk.gemm_unchecked(n, n, n, 1.0, a, n, 1, b, n, 1, 0.0, c, n, 1)  # noqa: E731
        ms = timed(call, steps, warm)
        flops = 2 * n ** 3
        e = {"ms": ms, **timed.last, "TFLOPS": flops / ms / 1e9,
             "roofline": roofline("f32", flops, ms, tr("f32_gemm_512"))}
        if oracle is not None:
            ah, bh = host(a), host(b)
            ch = np.empty(n * n, np.float32)

            def run(threads):
                oracle.port_gemm_f32(n, n, n, 1.0, ah, n, 1, bh, n, 1, 0.0, ch, n, 1, threads)
            sample = "the full 512^3 f32 product (all row-major) on the same inputs"
            e["cpu_baseline"] = cpu_legs({"all_cores": (run, flops, 3.0, sample),
                                          "serial": (run, flops, 3.0, sample)},
                                         "TFLOP/s", 1e12, oracle)
        workloads["f32_gemm_512"] = e

    # bf16 4096^3 with bf16 output: plain, and fused with a per-column bias and
    # ReLU (the epilogue's cost is the difference)
    if want("bf16_fused_4096"):
        n = 4096
        a = torch.randn(n * n, generator=g).to(torch.bfloat16).to(dev)
        b = torch.randn(n * n, generator=g).to(torch.bfloat16).to(dev)
        c = torch.empty(n * n, dtype=torch.bfloat16, device=dev)
        bias = torch.randn(n, generator=g).to(torch.bfloat16).to(dev)
        A, B = gk.MatRef.from_row_major(a, n, n), gk.MatRef(b, n, n, 1, n)
        C = gk.MatMut.from_row_major(c, n, n)
        plain = timed(lambda: gk.gemm(1.0, A, B, 0.0, C), steps, warm)
        fused = timed(lambda: gk.gemm_fused(1.0, A, B, 0.0, C, gk.Bias.PerCol(bias),
                                            gk.Activation.Relu), steps, warm)
        workloads["bf16_fused_4096"] = {"ms_plain": plain, "ms_fused": fused,
                                        "TFLOPS_fused": 2 * n ** 3 / fused / 1e9,
                                        "frac_bf16_peak": 2 * n ** 3 / (fused * 1e-3) / 2.5e15,
                                        "roofline": roofline("bf16", 2 * n ** 3, fused)}
        del a, b, c

    # prepacked weight at small batch (k = n = 2048, m = 8 and 64; A and C
    # column-major, f32 B row-major and i8 B column-major before packing), as
    # gemmkit's fixed-weight inference benchmark
    if want("packed_small_m"):
        k = n = 2048
        bf = torch.randn(k * n, generator=g).to(dev)
        pf = gk.prepack_rhs(gk.MatRef.from_row_major(bf, k, n))
        bi = i8(k * n)
        pi = gk.prepack_rhs_i8(gk.MatRef.from_col_major(bi, k, n))
        res = {}
        for m in (8, 64):
            af = torch.randn(m * k, generator=g).to(dev)
            cf = torch.empty(m * n, device=dev)
            ai = i8(m * k)
            ci = torch.empty(m * n, dtype=torch.int32, device=dev)
            t = {
                "f32_plain": lambda: gk.gemm(1.0, gk.MatRef.from_col_major(af, m, k),
                                             gk.MatRef.from_row_major(bf, k, n), 0.0,
                                             gk.MatMut.from_col_major(cf, m, n)),
                "f32_packed_b": lambda: gk.gemm_packed_b(1.0, gk.MatRef.from_col_major(af, m, k),
                                                         pf, 0.0, gk.MatMut.from_col_major(cf, m, n)),
                "i8_plain": lambda: gk.gemm_i8(1, gk.MatRef.from_col_major(ai, m, k),
                                               gk.MatRef.from_col_major(bi, k, n), 0,
                                               gk.MatMut.from_col_major(ci, m, n)),
                "i8_packed_b": lambda: gk.gemm_i8_packed_b(1, gk.MatRef.from_col_major(ai, m, k),
                                                           pi, 0, gk.MatMut.from_col_major(ci, m, n)),
            }
            for name, fn in t.items():
                ms = timed(fn, steps, warm)
                res[f"{name}_m{m}"] = {"us": ms * 1e3, "GFLOPS": 2 * m * n * k / ms / 1e6}
        workloads["packed_small_m"] = res
        del bf, pf, bi, pi

    # The vendor library on the same products and operand layouts, timed the
    # same way (not part of the default run; a comparison, never `value`):
    # torch._int_mm and torch.mm dispatch to hipBLASLt on this ROCm build.
    if args.only == "vendor":
        res = {}
        M = N = K = 4096
        ops = 2 * M * N * K
        a8 = i8(M * K).view(M, K)
        b8 = i8(N * K).view(N, K).t()  # column-major B via strides
        c8 = torch.empty(M, N, dtype=torch.int32, device=dev)
        ms = timed(lambda: torch._int_mm(a8, b8, out=c8), steps, warm)
        res["i8_gemm_4096"] = {"ms": ms, "TOPS": ops / ms / 1e9, **timed.last}
        g = torch.Generator().manual_seed(3)
        ab = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
        bbc = torch.randn(N, K, generator=g).to(torch.bfloat16).to(dev)  # B^T row-major
        bb = bbc.t()  # column-major B
        cf = torch.empty(M, N, dtype=torch.float32, device=dev)
        cb = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        ms = timed(lambda: torch.mm(ab, bb, out=cb), steps, warm)
        res["bf16_gemm_4096_bf16_out"] = {"ms": ms, "TFLOPS": ops / ms / 1e9, **timed.last}
        ms = timed(lambda: torch.mm(ab, bb, out_dtype=torch.float32, out=cf), steps, warm) \
            if "out_dtype" in torch.mm.__doc__ else None
        if ms is not None:
            res["bf16_gemm_4096_f32_out"] = {"ms": ms, "TFLOPS": ops / ms / 1e9, **timed.last}
        # this library on the same bf16 operands, same timing, for the side-by-side
        ms = timed(lambda: gk.gemm_unchecked(M, K, N, 1.0, ab.view(-1), K, 1, bbc.view(-1), 1, K,
                                             0.0, cb.view(-1), N, 1),
                   steps, warm)
        res["gemmkit_amd_bf16_gemm_4096_bf16_out"] = {"ms": ms, "TFLOPS": ops / ms / 1e9,
                                                      **timed.last}
        abf, cff = ab.view(-1), cf.view(-1)
        ms = timed(lambda: gk.gemm_bf16_f32out(1.0, gk.MatRef(abf, M, K, K, 1),
                                               gk.MatRef(bbc.view(-1), K, N, 1, K), 0.0,
                                               gk.MatMut(cff, M, N, N, 1)), steps, warm)
        res["gemmkit_amd_bf16_gemm_4096_f32_out"] = {"ms": ms, "TFLOPS": ops / ms / 1e9,
                                                     **timed.last}
        workloads["vendor"] = res

    # a plain elementwise kernel over 1 GiB in, 1 GiB out (reads and writes
    # each byte once): the calibration workload for the HBM byte counters
    if args.only == "copy_1gib":
        src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        ms = timed(lambda: torch.neg(src, out=dst), steps, warm)
        workloads["copy_1gib"] = {"ms": ms, "GBps": 2 * (1 << 30) / ms / 1e6}


if __name__ == "__main__":
    main()
