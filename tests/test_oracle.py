"""CPU tests that pin the oracle before anything is compared against it.

Each oracle function is checked against something that does not share its
code: the reference's literal known answers, fixtures written by pure-Python
models (tests/golden/make_golden.py), numpy's exact int64 / float64
arithmetic, torch's RNE bf16 conversion, brute force on tiny inputs, and the
ABFT checksum identity.  Planted-mistake checks confirm the comparisons would
catch a dropped term or a transposed operand.
"""
import json
import os
import struct

import numpy as np
import pytest

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


# ------------------------------------------------------------------- i8 GEMM

def test_i8_small_fixtures():
    for case in load("i8_gemm_small.json"):
        m, k, n = case["m"], case["k"], case["n"]
        a = np.array(case["a"], np.int8)
        b = np.array(case["b"], np.int8)
        c = np.array(case["c0"], np.int32)
        oracle.gemm_i8(m, k, n, case["alpha"], a, k, 1, b, n, 1, case["beta"], c, n, 1)
        assert c.tolist() == case["expected"], (m, k, n, case["alpha"], case["beta"])


def test_i8_generator_matches_fixture_inputs():
    case = load("i8_gemm_small.json")[2]
    m, k = case["m"], case["k"]
    assert oracle.rand_i8_100(0x100 + m * 7 + k, m * k).tolist() == case["a"]


def test_i8_wrap_kat():
    kat = load("kats.json")["i8_wrap"]
    a = np.array(kat["a"], np.int8)
    b = np.array(kat["b"], np.int8)
    c = np.array(kat["c0"], np.int32)
    oracle.gemm_i8(2, 2, 2, kat["alpha"], a, 2, 1, b, 2, 1, kat["beta"], c, 2, 1)
    acc = 127 * 127 * 2
    wrap = lambda v: (v + 2**31) % 2**32 - 2**31  # noqa: E731
    assert c.tolist() == [wrap(x + wrap(kat["alpha"] * acc)) for x in kat["c0"]]


@pytest.mark.parametrize("m,k,n", [(5, 9, 4), (64, 200, 33), (130, 1000, 70)])
def test_i8_vs_numpy_int64_all_layouts(m, k, n):
    a = oracle.rng_i8_full(m, m * k).reshape(m, k)
    b = oracle.rng_i8_full(n, k * n).reshape(k, n)
    ref = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.int32)
    for (rsa, csa, at) in ((k, 1, a), (1, m, a.T)):
        for (rsb, csb, bt) in ((n, 1, b), (1, k, b.T)):
            for (rsc, csc) in ((n, 1), (1, m)):
                c = np.zeros(m * n, np.int32)
                oracle.gemm_i8(m, k, n, 1, np.ascontiguousarray(at).ravel(), rsa, csa,
                               np.ascontiguousarray(bt).ravel(), rsb, csb, 0, c, rsc, csc)
                got = c.reshape(m, n) if rsc == n else c.reshape(n, m).T
                assert np.array_equal(got, ref)


def test_i8_abft_identity_and_planted_transpose():
    m, k, n = 40, 50, 30
    a = oracle.rng_i8_full(3, m * k)
    b = oracle.rng_i8_full(4, k * n)
    c = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a, k, 1, b, n, 1, 0, c, n, 1)
    assert np.array_equal(oracle.colsum_i32(m, n, c, n, 1), oracle.abft_i8(m, k, n, a, k, 1, b, n, 1))
    # a transposed operand (B read column-major by mistake) must break the identity
    bad = np.zeros(m * n, np.int32)
    kk = min(k, n)
    oracle.gemm_i8(m, kk, kk, 1, a, k, 1, b, 1, n, 0, bad, kk, 1)
    good = np.zeros(m * kk, np.int32)
    oracle.gemm_i8(m, kk, kk, 1, a, k, 1, b, n, 1, 0, good, kk, 1)
    assert not np.array_equal(bad[:m * kk], good)


def test_i8_negative_strides():
    m, k, n = 12, 9, 7
    a = oracle.rand_i8_100(5, m * k)
    b = oracle.rand_i8_100(6, k * n)
    fwd = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a, k, 1, b, n, 1, 0, fwd, n, 1)
    rev = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a, -k, 1, b, n, 1, 0, rev, n, 1, a_off=(m - 1) * k)
    assert np.array_equal(rev.reshape(m, n), fwd.reshape(m, n)[::-1])


# ------------------------------------------------------------------- requant

def test_requant_store_sweep_fixture():
    sw = load("requant_store_sweep.json")
    accs = sw["accumulators"]
    assert len(accs) == 104
    for case in sw["cases"]:
        s = struct.unpack("<f", struct.pack("<I", case["scale_f32_bits"]))[0]
        got = [oracle.requant_one(v, 0, s, case["zp"], case["lo"], case["hi"]) & 0xFF for v in accs]
        assert got == case["expected_low_byte"], case["scale_f32_bits"]


def test_requant_ties_kat():
    kat = load("kats.json")["requant_ties"]
    assert [oracle.requant_one(v, 0, kat["scale"], kat["zp"]) for v in kat["a"]] == kat["expected"]


def test_requant_bias_wraps_and_round_ne():
    # wrapping bias add (src/kernel/epilogue.rs:825): MAX + 1 wraps to MIN
    assert oracle.requant_one(2**31 - 1, 1, 1.0, 0) == -128
    assert oracle.requant_one(-2**31, -1, 1.0, 0) == 127
    # the 2^52 trick equals round-half-even, and passes large values through
    for x in (0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 4503599627370495.5, 1e300, -1e300, 0.49999999999999994):
        assert oracle.round_ne_f64(x) == (round(x) if abs(x) < 2**52 else x)
    # a planted round-half-up map would give 3 here; the fixture and the
    # oracle both say 2 (ties to even)
    planted = int(np.floor(5 * 0.5 + 0.5))
    assert planted == 3 and oracle.requant_one(5, 0, 0.5, 0) == 2


def test_requant_gemm_composition_vs_python():
    m, k, n = 9, 33, 11
    a = oracle.rng_i8_sym127(1, m * k)
    b = oracle.rng_i8_sym127(2, k * n)
    scales = np.array([0.003, 0.5, 1.0, 7.25, 0.0078125, 0.1, 0.01, 0.02, 0.3], np.float32)
    bias = np.array([(i * 977) % 2001 - 1000 for i in range(m)], np.int32)
    out = np.zeros(m * n, np.int8)
    oracle.gemm_i8_requant(m, k, n, a, k, 1, b, n, 1, 0.0, scales, 3, bias, 0, -128, 127,
                           out, n, 1)
    acc = a.reshape(m, k).astype(np.int64) @ b.reshape(k, n).astype(np.int64)
    for i in range(m):
        for j in range(n):
            x = float(int(acc[i, j]) + int(bias[i])) * float(scales[i])
            q = max(-128, min(127, round(x) + 3))
            assert out[i * n + j] == q
    # per-column axis: channel index follows j
    outc = np.zeros(m * n, np.uint8)
    sc = np.linspace(0.001, 0.05, n).astype(np.float32)
    oracle.gemm_i8_requant(m, k, n, a, k, 1, b, n, 1, 0.0, sc, 10, None, 1, 0, 255, outc, n, 1)
    for i in range(m):
        for j in range(n):
            q = max(0, min(255, round(float(int(acc[i, j])) * float(sc[j])) + 10))
            assert outc[i * n + j] == q


def test_requant_map_equals_fused():
    m, k, n = 20, 64, 17
    a = oracle.rng_i8_sym127(5, m * k)
    b = oracle.rng_i8_sym127(6, k * n)
    sc = np.linspace(0.001, 0.02, n).astype(np.float32)
    bias = np.arange(n, dtype=np.int32) * 1000 - 8000
    fused = np.zeros(m * n, np.int8)
    oracle.gemm_i8_requant(m, k, n, a, k, 1, b, n, 1, 0.0, sc, 0, bias, 1, 0, 127, fused, n, 1)
    acc = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a, k, 1, b, n, 1, 0, acc, n, 1)
    mapped = np.zeros(m * n, np.int8)
    oracle.requant_map(m, n, acc, n, 1, 0.0, sc, 0, bias, 1, 0, 127, mapped, n, 1)
    assert np.array_equal(fused, mapped)


# ---------------------------------------------------------------------- bf16

def test_bf16_rne_vs_torch():
    import torch
    x = np.concatenate([oracle.rng_normal(1, 20000) * 10.0 ** np.arange(-20, 20, 2).repeat(1000),
                        np.array([0.0, -0.0, 1.0, 65504.0, 3.4e38, -3.4e38, 1e-40, np.inf, -np.inf])])
    x = x.astype(np.float32)
    # exact ties: 1 + 2^-8 (tie, round to even 1.0) and 1 + 3*2^-8 (tie, round up)
    ties = np.array([1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, -(1 + 2.0 ** -8)], np.float32)
    x = np.concatenate([x, ties])
    got = oracle.bf16_bits(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert got[-3] == 0x3F80 and got[-2] == 0x3F82 and got[-1] == 0xBF80


def test_bf16_nan_rule():
    # NaN keeps its upper bits and is quieted: (bits >> 16) | 0x40
    for bits in (0x7F800001, 0x7FC00000, 0xFF812345, 0x7FFFFFFF):
        f = np.array([bits], np.uint32).view(np.float32)
        assert oracle.bf16_bits(f)[0] == ((bits >> 16) | 0x40)


# ------------------------------------------------------------ fused epilogue

def _bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def test_fused_map_reference_kats():
    # tests/epilogue/float.rs:274-358: a NaN value maps to +0 under ReLU and
    # LeakyReLU(0.25); a zero product under LeakyReLU(-0.5) is +0, not -0.
    nan = np.full((3, 5), np.nan, np.float32)
    assert (_bits(oracle.fused_map_f32(nan, act=1)) == 0).all()
    assert (_bits(oracle.fused_map_f32(nan, act=2, slope=0.25)) == 0).all()
    zeros = np.array([[0.0, -0.0, 0.0]], np.float32)
    assert (_bits(oracle.fused_map_f32(zeros, act=2, slope=-0.5)) == 0).all()
    assert (_bits(oracle.fused_map_f32(zeros, act=1)) == 0).all()
    # tests/epilogue/float.rs:361-395: the degenerate ReLU(0.5*C0 + bias[i]),
    # checked here against numpy's own float32 ops: the f32 sum of two f32
    # values equals the f64 sum rounded to f32, and max(x, 0) + 0 is ReLU with
    # -0 sent to +0.
    c0 = oracle.rng_unit(0xDE6E, 20 * 24).astype(np.float32).reshape(20, 24)
    bias = oracle.rng_unit(7, 20).astype(np.float32)
    base = np.float32(0.5) * c0
    got = oracle.fused_map_f32(base, bias, 0, 1)
    want = np.maximum((base.astype(np.float64) + bias[:, None]).astype(np.float32),
                      np.float32(0)) + np.float32(0)
    assert np.array_equal(_bits(got), _bits(want))


def test_fused_map_closed_forms():
    x = np.concatenate([oracle.rng_normal(3, 4000).astype(np.float32) *
                        np.float32(10.0) ** np.arange(-4, 4).repeat(500).astype(np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 3e38, -3e38],
                                 np.float32)]).reshape(1, -1)
    m, n = 3, x.shape[1]
    v = np.repeat(x, m, axis=0)
    brow = np.array([0.0, 1.5, -2.25], np.float32)
    bcol = oracle.rng_unit(9, n).astype(np.float32)
    for bias, dim in ((None, 0), (brow, 0), (bcol, 1)):
        if bias is None:
            y = v
        else:
            b = bias[:, None] if dim == 0 else bias[None, :]
            with np.errstate(invalid="ignore", over="ignore"):
                y = (v.astype(np.float64) + b).astype(np.float32)
        # no activation: the bias add alone
        assert np.array_equal(_bits(oracle.fused_map_f32(v, bias, dim, 0)), _bits(y))
        # ReLU
        with np.errstate(invalid="ignore"):
            want = np.where(np.isnan(y), np.float32(0), np.maximum(y, np.float32(0))) + np.float32(0)
        assert np.array_equal(_bits(oracle.fused_map_f32(v, bias, dim, 1)), _bits(want))
        # LeakyReLU: y for y > 0, the f32 product slope*y (then +0) for y < 0, +0
        # otherwise (zeros and NaN).  1e-45 * 0.25 underflows to -0 for a
        # negative input: a fused multiply-add would keep -0, the map gives +0.
        for slope in (0.1, 0.25, -0.5, 3.0):
            s = np.float32(slope)
            with np.errstate(invalid="ignore", over="ignore"):
                neg = (s * y) + np.float32(0)
                want = np.where(y > 0, y, np.where(y < 0, neg, np.float32(0))).astype(np.float32)
            got = oracle.fused_map_f32(v, bias, dim, 2, slope)
            assert np.array_equal(_bits(got), _bits(want)), (slope, dim)


def test_fused_map_bf16_widens_and_narrows_once():
    import torch
    v = (oracle.rng_normal(11, 6 * 50) * 4).astype(np.float32).reshape(6, 50)
    bias = oracle.bf16_bits(oracle.rng_unit(12, 50).astype(np.float32))
    slope = int(oracle.bf16_bits(np.array([0.1], np.float32))[0])
    for act in (0, 1, 2):
        got = oracle.fused_map_bf16(v, bias, 1, act, slope)
        f32 = oracle.fused_map_f32(v, oracle.bf16_to_f32(bias), 1, act,
                                   float(oracle.bf16_to_f32(np.array([slope]))[0]))
        want = torch.from_numpy(f32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(got, want)


# ----------------------------------------------------------------- f64 GEMM

def test_readme_kat_f64():
    kat = load("kats.json")["readme_2x2"]
    out = oracle.gemm_f64(2, 3, 2, 1.0, np.array(kat["a"], np.float32), 3, 1,
                          np.array(kat["b"], np.float32), 2, 1)
    assert out.ravel().tolist() == kat["expected"]


def test_f64_gemm_and_gemv_vs_numpy():
    m, k, n = 37, 50, 23
    a = oracle.rand_vec(1, m * k).astype(np.float32)
    b = oracle.rand_vec(2, k * n).astype(np.float32)
    c0 = oracle.rand_vec(3, m * n).astype(np.float32)
    got = oracle.gemm_f64(m, k, n, 0.5, a, k, 1, b, n, 1, -2.0, c0, n, 1)
    ref = 0.5 * (a.reshape(m, k).astype(np.float64) @ b.reshape(k, n).astype(np.float64)) \
        - 2.0 * c0.reshape(m, n).astype(np.float64)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    # beta == 0 never reads C: NaN in C0 must not leak
    nan_c = np.full(m * n, np.nan, np.float32)
    assert np.isfinite(oracle.gemm_f64(m, k, n, 1.0, a, k, 1, b, n, 1, 0.0, nan_c, n, 1)).all()
    y = oracle.gemv_f64(m, k, 1.0, a, k, 1, b[:k], 1)
    assert np.allclose(y, a.reshape(m, k).astype(np.float64) @ b[:k].astype(np.float64))


# ------------------------------------------------------------------ CPU port

@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (33, 17, 19), (100, 300, 50), (257, 1024, 129)])
@pytest.mark.parametrize("alpha,beta", [(1, 0), (3, -2), (1, 1)])
@pytest.mark.parametrize("row_major_c", [True, False])
def test_cpu_port_bit_exact(m, k, n, alpha, beta, row_major_c):
    a = oracle.rng_i8_full(10 + m, m * k)
    b = oracle.rng_i8_full(20 + n, k * n)
    rsc, csc = (n, 1) if row_major_c else (1, m)
    c0 = ((np.arange(m * n) % 7) - 3).astype(np.int32)
    want = c0.copy()
    oracle.gemm_i8(m, k, n, alpha, a, k, 1, b, 1, k, beta, want, rsc, csc)
    got = c0.copy()
    oracle.port_gemm_i8(m, k, n, alpha, a, k, 1, b, 1, k, beta, got, rsc, csc, threads=2)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("la,lb,lc", [("row", "col", "row"), ("col", "row", "col"),
                                      ("row+", "col+", "col+"), ("col+", "row+", "row")])
def test_cpu_port_strided_layouts(la, lb, lc):
    """The port from any operand strides (it packs them, as gemmkit does),
    i32 and requantized, against the closed forms: the GPU tests check large
    strided products against it."""
    from helpers import layout_strides, scatter
    rng = np.random.default_rng(0x5EED)
    for m, k, n in [(37, 53, 29), (64, 130, 70), (5, 300, 17)]:
        a = rng.integers(-128, 128, (m, k), dtype=np.int8)
        b = rng.integers(-128, 128, (k, n), dtype=np.int8)
        c0 = rng.integers(-1000, 1000, (m, n), dtype=np.int32)
        rsa, csa, al = layout_strides(m, k, la, 16)
        rsb, csb, bl = layout_strides(k, n, lb, 16)
        rsc, csc, cl = layout_strides(m, n, lc, 4)
        ab, bb = scatter(a, rsa, csa, al), scatter(b, rsb, csb, bl)
        cb = scatter(c0, rsc, csc, cl, fill=-77)
        want, got = cb.copy(), cb.copy()
        oracle.gemm_i8(m, k, n, 3, ab, rsa, csa, bb, rsb, csb, -1, want, rsc, csc)
        oracle.port_gemm_i8(m, k, n, 3, ab, rsa, csa, bb, rsb, csb, -1, got, rsc, csc, threads=2)
        assert np.array_equal(got, want)
        for axis in (0, 1):
            ch = n if axis else m
            sc = (1e-4 + rng.random(ch) * 1e-2).astype(np.float32)
            bias = rng.integers(-65536, 65537, ch, dtype=np.int32)
            q_want, q_got = np.zeros(cl, np.uint8), np.zeros(cl, np.uint8)
            oracle.gemm_i8_requant(m, k, n, ab, rsa, csa, bb, rsb, csb, 0.0, sc, 5, bias, axis,
                                   5, 127, q_want, rsc, csc)
            oracle.port_gemm_i8_requant(m, k, n, ab, rsa, csa, bb, rsb, csb, 0.0, sc, 5, bias,
                                        axis, 5, 127, q_got, rsc, csc, threads=2)
            assert np.array_equal(q_got, q_want)


def test_generators_are_reproducible():
    assert oracle.rng_next_u64(7, 3) == oracle.rng_next_u64(7, 3)
    x = oracle.rng_i8_full(5, 100000)
    assert x.min() == -128 and x.max() == 127
    y = oracle.rng_i8_sym127(5, 100000)
    assert y.min() == -127 and y.max() == 127
    u = oracle.rng_unit(5, 100000)
    assert -1 <= u.min() and u.max() < 1


# The other CPU-port families, pinned against the oracle's closed forms:
# bit-exact for the requantizing path, within the float bars for f32/bf16.

@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (33, 17, 19), (100, 300, 50), (70, 1024, 129)])
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("row_major_c", [True, False])
def test_cpu_port_requant_bit_exact(m, k, n, axis, row_major_c):
    a = oracle.rng_i8_sym127(30 + m, m * k)
    b = oracle.rng_i8_sym127(40 + n, k * n)  # B column-major (rsb = 1, csb = k)
    ch = m if axis == 0 else n
    scales = (1e-4 + (np.arange(ch) % 13) * 7.7e-4).astype(np.float32)
    bias = ((np.arange(ch) * 7919) % 131073 - 65536).astype(np.int32)
    rsc, csc = (n, 1) if row_major_c else (1, m)
    for zp, lo, hi in [(0, 0, 127), (3, -128, 127), (-5, -128, 127)]:
        want = np.zeros(m * n, np.int8)
        oracle.gemm_i8_requant(m, k, n, a, k, 1, b, 1, k, 0.0, scales, zp, bias, axis, lo, hi,
                               want, rsc, csc)
        got = np.zeros(m * n, np.int8)
        oracle.port_gemm_i8_requant(m, k, n, a, k, 1, b, 1, k, 0.0, scales, zp, bias, axis, lo,
                                    hi, got.view(np.uint8), rsc, csc, threads=2)
        assert np.array_equal(got, want), (zp, lo, hi)
        # the same with B prepacked once (no orientation swap: C as given)
        pb = oracle.PortPackedB(k, n, b, 1, k, threads=2)
        got2 = np.zeros(m * n, np.int8)
        oracle.port_gemm_i8_requant(m, k, n, a, k, 1, None, 0, 0, 0.0, scales, zp, bias, axis,
                                    lo, hi, got2.view(np.uint8), rsc, csc, threads=2, packed=pb)
        assert np.array_equal(got2, want), ("packed", zp, lo, hi)


def test_cpu_port_requant_per_tensor_scale():
    m, k, n = 40, 96, 30
    a = oracle.rng_i8_full(51, m * k)
    b = oracle.rng_i8_full(52, k * n)
    want = np.zeros(m * n, np.int8)
    oracle.gemm_i8_requant(m, k, n, a, k, 1, b, 1, k, 0.003, None, 1, None, 0, -128, 127, want,
                           n, 1)
    got = np.zeros(m * n, np.int8)
    oracle.port_gemm_i8_requant(m, k, n, a, k, 1, b, 1, k, 0.003, None, 1, None, 0, -128, 127,
                                got.view(np.uint8), n, 1, threads=3)
    assert np.array_equal(got, want)


def _rel_frob(got, ref):
    return np.linalg.norm(got.astype(np.float64) - ref) / np.linalg.norm(ref)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (33, 17, 19), (100, 300, 50), (257, 1024, 129),
                                   (512, 512, 512)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.5, 1.0), (2.0, -0.75)])
@pytest.mark.parametrize("row_major_c", [True, False])
def test_cpu_port_f32_within_tolerance(m, k, n, alpha, beta, row_major_c):
    a = oracle.rand_vec(60 + m, m * k).astype(np.float32)
    b = oracle.rand_vec(70 + n, k * n).astype(np.float32)
    rsc, csc = (n, 1) if row_major_c else (1, m)
    c0 = oracle.rand_vec(80, m * n).astype(np.float32)
    ref = oracle.gemm_f64(m, k, n, alpha, a, k, 1, b, n, 1, beta, c0.astype(np.float64), rsc,
                          csc)
    got = c0.copy()
    oracle.port_gemm_f32(m, k, n, alpha, a, k, 1, b, n, 1, beta, got, rsc, csc, threads=2)
    dense = got.reshape(m, n) if row_major_c else got.reshape(n, m).T
    assert _rel_frob(dense, ref) <= 1e-5


@pytest.mark.parametrize("batch,m,k,n", [(1, 33, 17, 19), (3, 64, 128, 64), (5, 100, 130, 70)])
def test_cpu_port_bf16_within_tolerance(batch, m, k, n):
    a = oracle.bf16_bits(oracle.rng_normal(90, batch * m * k).astype(np.float32))
    b = oracle.bf16_bits(oracle.rng_normal(91, batch * k * n).astype(np.float32))
    af = oracle.bf16_to_f32(a).astype(np.float64).reshape(batch, m, k)
    bf = oracle.bf16_to_f32(b).astype(np.float64).reshape(batch, n, k)  # B column-major
    alpha = 1.0 / np.sqrt(128.0)
    ref = alpha * np.einsum("zik,zjk->zij", af, bf)
    got = np.zeros(batch * m * n, np.float32)
    oracle.port_gemm_batched_bf16_f32out(batch, m, k, n, alpha, a, k, 1, m * k, b, 1, k, k * n,
                                         0.0, got, n, 1, m * n, threads=2)
    assert _rel_frob(got, ref.ravel()) <= 1e-5
    err = np.abs(got.astype(np.float64) - ref.ravel())
    assert (err <= 1e-2 * np.maximum(np.abs(ref.ravel()), 1e-3 * np.abs(ref).max())).all()


@pytest.mark.parametrize("rows,k", [(1, 1), (7, 33), (100, 1000), (1027, 4099)])
@pytest.mark.parametrize("beta", [0.0, 0.5])
def test_cpu_port_gemv_within_tolerance(rows, k, beta):
    a = oracle.rand_vec(100 + rows, rows * k).astype(np.float32)
    x = oracle.rand_vec(101, k).astype(np.float32)
    y0 = oracle.rand_vec(102, rows).astype(np.float32)
    ref = oracle.gemv_f64(rows, k, 1.25, a, k, 1, x, 1, beta, y0.astype(np.float64), 1)
    got = y0.copy()
    oracle.port_gemv_f32(rows, k, 1.25, a, k, x, beta, got, 1, threads=3)
    assert _rel_frob(got, ref) <= 1e-5


def test_generators_match_python_restatement():
    """The oracle's seeded streams (the inputs of the parity tests and the
    benchmark) against tests/golden/generators.json, written by a Python
    restatement of the reference's Rng (tests/epilogue/common.rs:16-34) and
    rand_vec (tests/oracle_common/mod.rs:121-132): integers exact, uniform
    floats bit-exact, Box-Muller normals within 4 ulp (libm cos/sin/log)."""
    path = os.path.join(os.path.dirname(__file__), "golden", "generators.json")
    g = json.load(open(path))
    for seed_s, want in g["next_u64"].items():
        assert oracle.rng_next_u64(int(seed_s), len(want)) == want, seed_s
    for seed_s, want in g["i8_full"].items():
        assert oracle.rng_i8_full(int(seed_s), len(want)).tolist() == want, seed_s
    for seed_s, want in g["i8_sym127"].items():
        assert oracle.rng_i8_sym127(int(seed_s), len(want)).tolist() == want, seed_s
    for seed_s, want in g["unit"].items():
        got = oracle.rng_unit(int(seed_s), len(want))
        assert [float.fromhex(w) for w in want] == got.tolist(), seed_s
    for seed_s, want in g["rand_vec"].items():
        got = oracle.rand_vec(int(seed_s), len(want))
        assert [float.fromhex(w) for w in want] == got.tolist(), seed_s
    for seed_s, want in g["normal"].items():
        got = oracle.rng_normal(int(seed_s), len(want))
        w = np.array([float.fromhex(x) for x in want])
        assert np.allclose(got, w, rtol=4 * 2.0 ** -52, atol=4 * 2.0 ** -52), seed_s
