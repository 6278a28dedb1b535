#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/ from pure-Python models.

Nothing here uses the oracle or the HIP library: the expected values come from
Python's exact integer arithmetic and IEEE-double float arithmetic, so they pin
the oracle (tests/test_oracle.py) independently.  Inputs follow the reference's
own tests:

* requant_store_sweep.json -- the adversarial accumulators and LCG tail of
  gemmkit/src/simd.rs:771-826 (LCG mul 6364136223846793005, add
  1442695040888963407, seed 0x123456789abcdef0, value = state >> 32 as i32)
  over scales {1.0, 0.1, 1e30, 1e-30, 0.0078125} (rounded to f32, the API's
  scale type), zero points {0, -128, 127} and bands (-128, 127), (0, 255).
  Expected = low byte of clamp(sat_i64(round_half_even(acc * scale)) + zp, lo, hi)
  (the independent model of simd.rs:739-743 and tests/epilogue/requant.rs:12-22).
* i8_gemm_small.json -- rand_i8 (tests/correctness/common.rs:137-147) operands,
  C0 = (x % 7) - 3 (tests/correctness/int8.rs:28), expected by Python loops
  with exact integers, wrapped to i32, for the (alpha, beta) pairs of
  tests/correctness/int8.rs:27.
* kats.json -- literal known answers copied from the reference's tests
  (README 2x2, requant ties, the i8 wrap case).

Run: python tests/golden/make_golden.py
"""
import json
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))
M64 = (1 << 64) - 1


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def wrap32(v: int) -> int:
    return (v + 2**31) % 2**32 - 2**31


def requant_model(acc: int, scale: float, zp: int, lo: int, hi: int) -> int:
    x = float(acc) * scale                 # one IEEE double multiply
    r = round(x)                           # Python round(): ties to even, exact int
    r = max(-2**63, min(2**63 - 1, r))     # Rust's saturating f64 -> i64
    q = max(-2**63, min(2**63 - 1, r + zp))
    q = max(lo, min(hi, q))
    return q & 0xFF


def lcg_values():
    vals = [-2**31, -2**31 + 1, -1, 0, 1, 1 << 30, 2**31 - 2, 2**31 - 1]
    s = 0x123456789ABCDEF0
    for _ in range(96):
        s = (s * 6364136223846793005 + 1442695040888963407) & M64
        v = s >> 32
        vals.append(v - 2**32 if v >= 2**31 else v)
    return vals


def sweep():
    vals = lcg_values()
    cases = []
    for s in (1.0, 0.1, 1e30, 1e-30, 0.0078125):
        sf = f32(s)
        for zp in (0, -128, 127):
            for lo, hi in ((-128, 127), (0, 255)):
                cases.append({"scale_f32_bits": struct.unpack("<I", struct.pack("<f", sf))[0],
                              "zp": zp, "lo": lo, "hi": hi,
                              "expected_low_byte": [requant_model(v, sf, zp, lo, hi) for v in vals]})
    return {"accumulators": vals, "cases": cases}


def rand_i8(n: int, seed: int):
    s = (seed + 0x9E3779B97F4A7C15) & M64
    out = []
    for _ in range(n):
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        out.append((s >> 24) % 201 - 100)
    return out


def i8_small():
    out = []
    for (m, k, n) in ((1, 1, 1), (3, 4, 5), (7, 13, 5), (16, 8, 7)):
        a = rand_i8(m * k, 0x100 + m * 7 + k)
        b = rand_i8(k * n, 0x200 + n * 3 + k)
        c0 = [(x % 7) - 3 for x in range(m * n)]
        for alpha, beta in ((1, 0), (1, 1), (3, -2), (0, 3), (100000, 7)):
            c = []
            for i in range(m):
                for j in range(n):
                    acc = sum(a[i * k + p] * b[p * n + j] for p in range(k))
                    if alpha == 0:
                        v = 0 if beta == 0 else wrap32(beta * c0[i * n + j])
                    else:
                        v = wrap32(beta * c0[i * n + j] + wrap32(alpha * wrap32(acc)))
                    c.append(v)
            out.append({"m": m, "k": k, "n": n, "alpha": alpha, "beta": beta, "a": a, "b": b,
                        "c0": c0, "expected": c})
    return out


def kats():
    return {
        # README.md:55-71, src/lib.rs:9-25
        "readme_2x2": {"a": [1, 2, 3, 4, 5, 6], "b": [7, 8, 9, 10, 11, 12],
                       "expected": [58.0, 64.0, 139.0, 154.0]},
        # tests/epilogue/requant.rs:253-272
        "requant_ties": {"a": [1, 3, 5, 7, -1, -3], "scale": 0.5, "zp": 0,
                         "expected": [0, 2, 2, 4, 0, -2]},
        # tests/correctness/int8.rs:198-232
        "i8_wrap": {"a": [127] * 4, "b": [127] * 4,
                    "c0": [1000000, -2000000, 3000000, -4000000], "alpha": 100000, "beta": 1},
    }


def main():
    with open(os.path.join(HERE, "requant_store_sweep.json"), "w") as f:
        json.dump(sweep(), f, separators=(",", ":"))
    with open(os.path.join(HERE, "i8_gemm_small.json"), "w") as f:
        json.dump(i8_small(), f, separators=(",", ":"))
    with open(os.path.join(HERE, "kats.json"), "w") as f:
        json.dump(kats(), f, indent=1)


if __name__ == "__main__":
    main()
