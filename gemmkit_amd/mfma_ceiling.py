"""Measures the matrix cores' practical ceiling on the current device.

Runs gk_debug_mfma_ceiling (gemmkit_amd/csrc/ceiling.hip): every CU issues
nothing but back-to-back MFMAs on random register operands, int8 and bf16, on
the 32x32 instructions (v_mfma_i32_32x32x32_i8, v_mfma_f32_32x32x16_bf16) and
the 16x16 ones (v_mfma_i32_16x16x64_i8, v_mfma_f32_16x16x32_bf16), after
about a second of the same load so the clocks settle.  The rate it reaches,
and the shader clock the chip holds meanwhile, bound what a GEMM kernel built
on that instruction can do on this part: MI355X is power-limited under
sustained matrix-core load, so the ceiling sits below the published dense
peaks (5.0 POP/s int8, 2.5 PFLOP/s bf16 at 2.4 GHz), and lower for the 32x32
instructions, which draw more power per operation.

Usage: python -m gemmkit_amd.mfma_ceiling [--json OUT]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json

from . import _lib

PEAK = {"int8": 5.0e15, "bf16": 2.5e15}
CODES = {("int8", 32): 0, ("bf16", 32): 1, ("int8", 16): 2, ("bf16", 16): 3}
SHAPES = {("int8", 32): "32x32x32", ("bf16", 32): "32x32x16", ("int8", 16): "16x16x64",
          ("bf16", 16): "16x16x32"}


def measure(kind: str, mfma: int = 32, iters: int = 100_000, launches: int = 40,
            wgs_per_cu: int = 1):
    ops, clk = C.c_double(), C.c_double()
    rc = _lib.lib().gk_debug_mfma_ceiling(CODES[(kind, mfma)], iters, wgs_per_cu, launches,
                                          C.byref(ops), C.byref(clk))
    if rc != 0:
        raise RuntimeError(f"gk_debug_mfma_ceiling failed: {rc}")
    return {"kind": kind, "instruction": SHAPES[(kind, mfma)], "wgs_per_cu": wgs_per_cu,
            "iters": iters, "launches": launches, "ops_per_s": ops.value,
            "clock_ghz": clk.value, "frac_of_published_peak": ops.value / PEAK[kind]}


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--json", default=None)
    args = p.parse_args()
    import torch
    torch.cuda.init()
    rows = [measure(k, s) for s in (32, 16) for k in ("int8", "bf16")]
    for r in rows:
        unit = "POP/s" if r["kind"] == "int8" else "PFLOP/s"
        print(f"{r['kind']:5s} {r['instruction']:9s} {r['wgs_per_cu']} wg/CU: "
              f"{r['ops_per_s'] / 1e15:.3f} {unit} "
              f"at {r['clock_ghz']:.3f} GHz = {100 * r['frac_of_published_peak']:.1f}% of the "
              f"published peak", flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump(rows, f, indent=1)


if __name__ == "__main__":
    main()
