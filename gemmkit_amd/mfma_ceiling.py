"""Measures the matrix cores' practical ceiling on the current device.

Runs gk_debug_mfma_ceiling (gemmkit_amd/csrc/ceiling.hip): every CU issues
nothing but back-to-back MFMAs on random register operands, int8
(v_mfma_i32_32x32x32_i8) and bf16 (v_mfma_f32_32x32x16_bf16), after about a
second of the same load so the clocks settle.  The rate it reaches, and the
shader clock the chip holds meanwhile, bound what any GEMM kernel can do on
this part: MI355X is power-limited under sustained matrix-core load, so the
ceiling sits below the published dense peaks (5.0 POP/s int8, 2.5 PFLOP/s
bf16 at 2.4 GHz).

Usage: python -m gemmkit_amd.mfma_ceiling [--json OUT]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json

from . import _lib

PEAK = {"int8": 5.0e15, "bf16": 2.5e15}


def measure(kind: str, iters: int = 100_000, launches: int = 40, wgs_per_cu: int = 1):
    ops, clk = C.c_double(), C.c_double()
    rc = _lib.lib().gk_debug_mfma_ceiling(0 if kind == "int8" else 1, iters, wgs_per_cu,
                                          launches, C.byref(ops), C.byref(clk))
    if rc != 0:
        raise RuntimeError(f"gk_debug_mfma_ceiling failed: {rc}")
    return {"kind": kind, "wgs_per_cu": wgs_per_cu, "iters": iters, "launches": launches,
            "ops_per_s": ops.value, "clock_ghz": clk.value,
            "frac_of_published_peak": ops.value / PEAK[kind]}


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--json", default=None)
    args = p.parse_args()
    import torch
    torch.cuda.init()
    rows = [measure(k) for k in ("int8", "bf16")]
    for r in rows:
        unit = "POP/s" if r["kind"] == "int8" else "PFLOP/s"
        print(f"{r['kind']:5s} {r['wgs_per_cu']} wg/CU: {r['ops_per_s'] / 1e15:.3f} {unit} "
              f"at {r['clock_ghz']:.3f} GHz = {100 * r['frac_of_published_peak']:.1f}% of the "
              f"published peak", flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump(rows, f, indent=1)


if __name__ == "__main__":
    main()
