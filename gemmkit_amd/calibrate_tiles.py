"""Measure the matrix-core tile shapes on a set of GEMM shapes and fit the
tile-choice cost model of ``csrc/capi.cpp`` (``pick_tile``) to the timings.

Maintenance tool, not part of the library's call path.  On a GPU box:

    python -m gemmkit_amd.calibrate_tiles --measure calib.json
    python -m gemmkit_amd.calibrate_tiles --fit calib.json        # CPU is enough

``--measure`` times every shape with each tile forced (GEMMKIT_HIP_TILE) and
with the library's own choice ("auto"), one HIP-graph replay of 12 calls per
point.  ``--fit`` fits per-tile efficiencies (with a factor for int8 inputs),
epilogue overlap, epilogue speeds (plain and requantizing), per-output-kind
epilogue costs, the per-tile latency and the f32 rate by least squares on log
time, then refines them to minimise the regret of the picks (time of the
predicted best tile over the measured best), and prints the constants and each shape's pick.
"""
from __future__ import annotations

import argparse
import json
import os

TILES = {"256x256": (256, 256, 1), "256x256w8": (256, 256, 1), "256x128o2": (256, 128, 2),
         "256x128": (256, 128, 1), "128x128": (128, 128, 2), "64x64": (64, 64, 2),
         "256x256k128": (256, 256, 1), "256x256w8k128": (256, 256, 1),
         "256x256w8m16": (256, 256, 1)}
# The 16x16-MFMA tile: no f32-input variant, and the library keeps bf16
# contractions of at most 256 bytes (the streaming kernel's, to which the
# 32x32 tiles are bit-identical) off it; it is not measured on f32 shapes
# and not fitted or picked where the library would not take it.
M16 = "256x256w8m16"


def tiles_for(meta, measuring=False):
    out = []
    for t in TILES:
        if t == M16 and meta.get("f32_in"):
            continue
        if (t == M16 and not measuring and meta["kind"] in ("f32", "bf16") and
                not meta.get("f32_in") and meta["K"] <= 256):
            continue
        out.append(t)
    return out
KINDS = ["i32", "q8", "f32", "bf16"]
CUS = 256


def measure(out_path: str) -> None:
    import torch
    import gemmkit_amd as gk
    gk.set_synchronous(False)
    dev = torch.device("cuda:0")

    def timed(fn, steps=12):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            with torch.cuda.graph(gr, stream=side):
                for _ in range(steps):
                    fn()
        torch.cuda.current_stream().wait_stream(side)
        gr.replay()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        gr.replay()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / steps * 1e3

    g = torch.Generator().manual_seed(0)

    def i8(n):
        return torch.randint(-127, 128, (n,), dtype=torch.int8, generator=g).to(dev)

    cases = {}

    def add_i8(name, M, N, K, q8=False):
        a, b = i8(M * K), i8(N * K)
        if q8:
            bias = torch.randint(-65536, 65537, (N,), dtype=torch.int32, generator=g).to(dev)
            sc = (1e-4 + torch.rand(N, generator=g) * 1e-2).to(dev)
            c = torch.empty(M * N, dtype=torch.int8, device=dev)
            fn = lambda: gk.gemm_i8_requant_unchecked(M, K, N, a, K, 1, b, 1, K, 0.0, sc, 0,  # noqa: E731
                                                      bias, c, N, 1, axis=1, relu=True)
        else:
            c = torch.empty(M * N, dtype=torch.int32, device=dev)
            fn = lambda: gk.gemm_i8_unchecked(M, K, N, 1, a, K, 1, b, 1, K, 0, c, N, 1)  # noqa: E731
        cases[name] = (dict(M=M, N=N, K=K, batch=1, kind="q8" if q8 else "i32"), fn)

    def add_bf(name, M, N, K, batch=1, out="f32"):
        a = torch.randn(batch * M * K, generator=g).to(torch.bfloat16).to(dev)
        b = torch.randn(batch * N * K, generator=g).to(torch.bfloat16).to(dev)
        A, B = gk.MatRef.from_row_major(a, M, K), gk.MatRef(b, K, N, 1, K)
        if out == "f32":
            c = torch.empty(batch * M * N, dtype=torch.float32, device=dev)
            fn = lambda: gk.gemm_batched_bf16_f32out(batch, 1.0, A, M * K, B, N * K, 0.0,  # noqa: E731
                                                     gk.MatMut.from_row_major(c, M, N), M * N)
        else:
            c = torch.empty(batch * M * N, dtype=torch.bfloat16, device=dev)
            fn = lambda: gk.gemm_batched(batch, 1.0, A, M * K, B, N * K, 0.0,  # noqa: E731
                                         gk.MatMut.from_row_major(c, M, N), M * N)
        cases[name] = (dict(M=M, N=N, K=2 * K, batch=batch, kind=out), fn)

    def add_f32(name, M, N, K):
        a = torch.randn(M * K, generator=g).to(dev)
        b = torch.randn(N * K, generator=g).to(dev)
        c = torch.empty(M * N, device=dev)
        cases[name] = (dict(M=M, N=N, K=4 * K, batch=1, kind="f32", f32_in=True),
                       lambda: gk.gemm_unchecked(M, K, N, 1.0, a, K, 1, b, 1, K, 0.0, c, N, 1))

    add_i8("i8_4096", 4096, 4096, 4096)
    add_i8("i8_layer_q8", 2048, 11008, 4096, q8=True)
    add_i8("i8_layer_i32", 2048, 11008, 4096)
    add_i8("i8_8192x8192x1024", 8192, 8192, 1024)
    add_i8("i8_1024x1024x8192", 1024, 1024, 8192)
    add_i8("i8_3000x5000x2000", 3000, 5000, 2000)
    add_i8("i8_q8_4096", 4096, 4096, 4096, q8=True)
    add_bf("bf16_4096", 4096, 4096, 4096)
    add_bf("bf16_attn", 512, 512, 128, batch=64)
    add_bf("bf16_layer_bf16out", 2048, 11008, 4096, out="bf16")
    add_bf("bf16_2048_bf16out", 2048, 2048, 2048, out="bf16")
    add_f32("f32_2048", 2048, 2048, 2048)
    add_f32("f32_1024", 1024, 1024, 1024)
    # the rests a tail split launches (one short round of the CUs), and f32
    # with many tiles
    add_i8("i8_rest_q8", 2048, 2816, 4096, q8=True)
    add_i8("i8_rest_i32", 2048, 2816, 4096)
    add_bf("bf16_rest_bf16out", 2048, 2816, 4096, out="bf16")
    add_f32("f32_4096x4096x1024", 4096, 4096, 1024)
    res = {}
    for name, (meta, fn) in cases.items():
        row = {}
        for t in tiles_for(meta, measuring=True) + ["auto"]:
            if t == "auto":
                os.environ.pop("GEMMKIT_HIP_TILE", None)
            else:
                os.environ["GEMMKIT_HIP_TILE"] = t
            row[t] = round(timed(fn), 2)
        os.environ.pop("GEMMKIT_HIP_TILE", None)
        res[name] = dict(meta=meta, us=row)
        print(name, json.dumps(row), flush=True)
    with open(out_path, "w") as f:
        json.dump(res, f, indent=1)


def fit(path: str) -> None:
    import numpy as np
    from scipy.optimize import least_squares
    data = json.load(open(path))
    tn = list(TILES)
    occ2 = [t for t in tn if TILES[t][2] == 2]
    pts = [(d["meta"], t, d["us"][t]) for d in data.values() for t in tiles_for(d["meta"])]

    nt = len(tn)

    def unpack(p):
        i = 0
        e1 = dict(zip(tn, p[i:i + nt])); i += nt
        e2 = dict(zip(occ2, p[i:i + len(occ2)])); i += len(occ2)
        hd = dict(zip(tn, p[i:i + nt])); i += nt
        ce = dict(zip(KINDS, p[i:i + 4])); i += 4
        lat, rf, s = p[i], p[i + 1], p[i + 2]; i += 3
        es = dict(zip(tn, [1.0] + list(p[i:i + nt - 1]))); i += nt - 1
        eq = dict(zip(tn, [1.0] + list(p[i:i + nt - 1]))); i += nt - 1
        ei = dict(zip(tn, [1.0] + list(p[i:i + nt - 1])))
        return e1, e2, hd, ce, lat, rf, s, es, eq, ei

    def model(p, meta, t):
        e1, e2, hd, ce, lat, rf, s, es, eq, ei = unpack(p)
        bm, bn, occ = TILES[t]
        ntile = -(-meta["M"] // bm) * -(-meta["N"] // bn) * meta["batch"]
        per = -(-ntile // CUS)
        eff = (e1[t] if min(per, occ) == 1 else e2[t]) * (ei[t] if meta["kind"] in ("i32", "q8") else 1.0)
        area = bm * bn
        kf = max(meta["K"], 64) / 4096.0 * (rf if meta.get("f32_in") else 1.0)
        exposed = per - hd[t] * (per - 1)
        speed = eq[t] if meta["kind"] == "q8" else es[t]
        return s * (per * area * kf / eff + (area * ce[meta["kind"]] * speed + lat) * exposed)

    def resid(p):
        return [np.log(model(p, m, t) / us) for m, t, us in pts]

    def pick(p, meta):
        # pick_tile's rule: candidates in order, a later one must be 0.1% cheaper
        best, bt = float("inf"), None
        for t in tiles_for(meta):
            c = model(p, meta, t)
            if c < best * 0.999:
                best, bt = c, t
        return bt

    def regret(p):
        tot = 0.0
        for d in data.values():
            tot += d["us"][pick(p, d["meta"])] / min(d["us"][t] for t in tiles_for(d["meta"])) - 1
        return tot

    p0 = [0.7] * nt + [0.5] * len(occ2) + [0.5] * nt + [0.3, 0.5, 0.3, 0.2, 4000, 4, 0.0005] + \
        [1.0] * (3 * nt - 3)
    lo = [0.05] * (nt + len(occ2)) + [0.0] * nt + [0.0] * 4 + [0, 1, 1e-5] + [0.2] * (2 * nt - 2) + \
        [0.7] * (nt - 1)
    hi = [1.0] * (nt + len(occ2)) + [1.0] * nt + [3.0] * 4 + [50000, 30, 1e-2] + [3.0] * (2 * nt - 2) + \
        [1.3] * (nt - 1)
    start = least_squares(resid, p0, bounds=(lo, hi)).x
    obj = lambda p: regret(p) + 0.2 * np.sqrt(np.mean(np.square(resid(p))))  # noqa: E731
    best, bo = start, obj(start)
    for seed in range(6):  # random-walk refinements from the least-squares fit
        rng = np.random.default_rng(seed)
        cur, co = start.copy(), obj(start)
        for _ in range(5000):
            q = cur.copy()
            k = rng.integers(len(q))
            q[k] = np.clip(q[k] * np.exp(rng.normal(0, 0.2)), lo[k], hi[k])
            o = obj(q)
            if o < co:
                cur, co = q, o
        if co < bo:
            best, bo = cur, co
    e1, e2, hd, ce, lat, rf, s, es, eq, ei = unpack(best)
    r6 = lambda x: round(float(x), 6)  # noqa: E731
    print("eff (one tile / two sharing a CU):", {t: (r6(e1[t]), r6(e2.get(t, e1[t]))) for t in tn})
    print("hide:", {t: r6(hd[t]) for t in tn})
    print("epilogue speed:", {t: r6(es[t]) for t in tn})
    print("requantizing epilogue speed:", {t: r6(eq[t]) for t in tn})
    print("i8 efficiency factor:", {t: r6(ei[t]) for t in tn})
    print("c_epi:", {k: r6(v) for k, v in ce.items()}, "latency", round(float(lat), 3),
          "f32 rate", r6(rf))
    print("regret", round(regret(best), 4), "rms log error",
          round(float(np.sqrt(np.mean(np.square(resid(best))))), 4))
    for name, d in data.items():
        pred = pick(best, d["meta"])
        bm = min(tiles_for(d["meta"]), key=lambda t: d["us"][t])
        print(f"{name:22s} pick {pred:10s} {d['us'][pred]:8.2f} us   best {bm:10s} "
              f"{d['us'][bm]:8.2f} us")


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--measure", metavar="OUT_JSON")
    ap.add_argument("--fit", metavar="IN_JSON")
    args = ap.parse_args()
    if args.measure:
        measure(args.measure)
    if args.fit:
        fit(args.fit)
