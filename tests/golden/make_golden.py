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
* generators.json -- the seeded streams the tests and the benchmark draw their
  inputs from, restated in Python from the reference's definitions: Rng, the
  xorshift* of tests/epilogue/common.rs:16-34 (next_u64, unit), with the i8
  fills built on it (full range: next % 256 - 128; make_i8 of
  tests/epilogue/requant.rs:25-30: next % 255 - 127); rand_vec of
  tests/oracle_common/mod.rs:121-132 (xorshift64 13/7/17 from seed + the
  golden-ratio constant, 2u - 1); and the Box-Muller normals over the Rng
  stream (this build's own, u1 = (next >> 11 + 1) / 2^53, u2 = (next >> 11) /
  2^53, r = sqrt(-2 ln u1), then r cos(2 pi u2) and r sin(2 pi u2)).

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


class Rng:
    """xorshift* of tests/epilogue/common.rs:16-34."""

    def __init__(self, seed: int):
        self.s = (seed | 1) & M64

    def next_u64(self) -> int:
        x = self.s
        x ^= x >> 12
        x ^= (x << 25) & M64
        x ^= x >> 27
        self.s = x
        return (x * 0x2545F4914F6CDD1D) & M64

    def unit(self) -> float:
        return (self.next_u64() >> 11) / float(1 << 53) * 2.0 - 1.0


def rand_vec(n: int, seed: int):
    s = (seed + 0x9E3779B97F4A7C15) & M64
    out = []
    for _ in range(n):
        s ^= (s << 13) & M64
        s ^= s >> 7
        s ^= (s << 17) & M64
        out.append(2.0 * ((s >> 11) / float(1 << 53)) - 1.0)
    return out


def normals(n: int, seed: int):
    import math
    r_ = Rng(seed)
    out = []
    while len(out) < n:
        u1 = ((r_.next_u64() >> 11) + 1.0) / float(1 << 53)
        u2 = (r_.next_u64() >> 11) / float(1 << 53)
        r = math.sqrt(-2.0 * math.log(u1))
        out.append(r * math.cos(2 * math.pi * u2))
        out.append(r * math.sin(2 * math.pi * u2))
    return out[:n]


def generators():
    out = {"next_u64": {}, "i8_full": {}, "i8_sym127": {}, "unit": {}, "rand_vec": {},
           "normal": {}}
    for seed in (0, 1, 2, 7, 0x123456789ABCDEF, 2**64 - 2):
        r = Rng(seed)
        out["next_u64"][str(seed)] = [r.next_u64() for _ in range(64)]
        r = Rng(seed)
        out["i8_full"][str(seed)] = [r.next_u64() % 256 - 128 for _ in range(300)]
        r = Rng(seed)
        out["i8_sym127"][str(seed)] = [r.next_u64() % 255 - 127 for _ in range(300)]
        r = Rng(seed)
        out["unit"][str(seed)] = [r.unit().hex() for _ in range(64)]
        out["rand_vec"][str(seed)] = [v.hex() for v in rand_vec(64, seed)]
        out["normal"][str(seed)] = [v.hex() for v in normals(63, seed)]
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
    with open(os.path.join(HERE, "generators.json"), "w") as f:
        json.dump(generators(), f, separators=(",", ":"))


if __name__ == "__main__":
    main()
