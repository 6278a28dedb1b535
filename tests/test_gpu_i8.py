"""GPU parity: i8 -> i32 GEMM through the C ABI against the oracle, bit-exact.

Shapes, layouts and alpha/beta pairs follow gemmkit's own i8 suite
(tests/correctness/int8.rs:8-51 correctness_i8, :198-232 wrap, :278-316
negative strides) plus larger and ragged shapes that cross the MFMA tile
edges; 4096^3 (the benchmark shape) is checked by sampled rows and an exact
column-checksum identity.
"""
import numpy as np
import pytest

import gemmkit_amd as gk
import oracle
from helpers import gather, layout_strides, scatter, to_dev

pytestmark = pytest.mark.gpu

REF_SHAPES = [(1, 1, 1), (3, 4, 5), (16, 8, 7), (32, 32, 32), (33, 17, 19), (40, 33, 28),
              (64, 80, 48), (65, 64, 64), (128, 96, 112)]
REF_AB = [(1, 0), (1, 1), (3, -2), (0, 3)]


def run_case(dev, m, k, n, alpha, beta, la, lb, lc, seed=0, gen=oracle.rand_i8_100, pad=3):
    a = gen(0x100 + seed + m * 7 + k, m * k).reshape(m, k)
    b = gen(0x200 + seed + n * 3 + k, k * n).reshape(k, n)
    c0 = ((np.arange(m * n) % 7) - 3).astype(np.int32).reshape(m, n)
    rsa, csa, la_len = layout_strides(m, k, la, pad)
    rsb, csb, lb_len = layout_strides(k, n, lb, pad)
    rsc, csc, lc_len = layout_strides(m, n, lc, pad)
    abuf = scatter(a, rsa, csa, la_len)
    bbuf = scatter(b, rsb, csb, lb_len)
    cbuf = scatter(c0, rsc, csc, lc_len, fill=-77)
    want = cbuf.copy()
    oracle.gemm_i8(m, k, n, alpha, abuf, rsa, csa, bbuf, rsb, csb, beta, want, rsc, csc)
    ad, bd, cd = to_dev(abuf, dev), to_dev(bbuf, dev), to_dev(cbuf, dev)
    gk.gemm_i8(alpha, gk.MatRef(ad, m, k, rsa, csa), gk.MatRef(bd, k, n, rsb, csb), beta,
               gk.MatMut(cd, m, n, rsc, csc))
    got = cd.cpu().numpy()
    if not np.array_equal(got, want):
        bad = np.flatnonzero(got != want)
        raise AssertionError(f"{m}x{k}x{n} a={alpha} b={beta} {la}/{lb}/{lc}: "
                             f"{bad.size} mismatches, first at {bad[:5]} got {got[bad[:5]]} "
                             f"want {want[bad[:5]]}")


@pytest.mark.parametrize("m,k,n", REF_SHAPES)
@pytest.mark.parametrize("alpha,beta", REF_AB)
def test_reference_suite_layout(dev, m, k, n, alpha, beta):
    # correctness_i8: row-major A, col-major B, row-major C
    run_case(dev, m, k, n, alpha, beta, "row", "col", "row")


@pytest.mark.parametrize("m,k,n", [(33, 17, 19), (65, 64, 64), (200, 130, 175), (384, 96, 320)])
@pytest.mark.parametrize("la,lb,lc", [("col", "col", "col"), ("row", "row", "row"),
                                      ("col", "row", "col"), ("row+", "col+", "col+"),
                                      ("col+", "row+", "row+")])
def test_layouts(dev, m, k, n, la, lb, lc):
    run_case(dev, m, k, n, 2, 3, la, lb, lc, seed=5)


@pytest.mark.parametrize("m,k,n", [(257, 256, 255), (512, 512, 512), (300, 1000, 700),
                                   (1024, 4096, 1024), (9, 4096, 777), (777, 4096, 9),
                                   (8, 512, 1000), (1000, 512, 8), (1, 4096, 14336)])
def test_tile_edges_full_range(dev, m, k, n):
    # full i8 range [-128, 127] (the benchmark's generator), canonical layout
    run_case(dev, m, k, n, 1, 0, "row", "col", "row", gen=oracle.rng_i8_full)


def test_wraps_on_overflow(dev):
    # tests/correctness/int8.rs:198-232: all-127 2x2, alpha = 100000 overflows i32
    a = np.full(4, 127, np.int8)
    b = np.full(4, 127, np.int8)
    c0 = np.array([1_000_000, -2_000_000, 3_000_000, -4_000_000], np.int32)
    alpha, beta = 100_000, 1
    acc = 127 * 127 * 2
    assert alpha * acc > 2**31 - 1  # the setup really overflows

    def wrap(v):
        return (v + 2**31) % 2**32 - 2**31

    want = np.array([wrap(beta * int(c) + wrap(alpha * acc)) for c in c0], np.int32)
    cd = to_dev(c0, dev)
    gk.gemm_i8(alpha, gk.MatRef.from_row_major(to_dev(a, dev), 2, 2),
               gk.MatRef.from_row_major(to_dev(b, dev), 2, 2), beta,
               gk.MatMut.from_row_major(cd, 2, 2))
    assert np.array_equal(cd.cpu().numpy(), want)


def test_negative_stride_unchecked(dev):
    # tests/correctness/int8.rs:278-316: A's base at its last row, rsa = -k
    m, k, n = 12, 9, 7
    a = oracle.rand_i8_100(5, m * k)
    b = oracle.rand_i8_100(6, k * n)
    want = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a, k, 1, b, n, 1, 0, want, n, 1)
    ad, bd = to_dev(a, dev), to_dev(b, dev)
    cd = to_dev(np.zeros(m * n, np.int32), dev)
    gk.gemm_i8_unchecked(m, k, n, 1, ad, -k, 1, bd, n, 1, 0, cd, n, 1, a_off=(m - 1) * k)
    got = cd.cpu().numpy().reshape(m, n)
    assert np.array_equal(got, want.reshape(m, n)[::-1])


def test_degenerate_k0_and_alpha0(dev):
    m, n = 5, 6
    c0 = np.arange(m * n, dtype=np.int32) - 7
    for alpha, beta, k in [(1, 0, 0), (1, 1, 0), (1, 3, 0), (0, -2, 4), (0, 0, 4)]:
        cd = to_dev(c0, dev)
        a = to_dev(np.ones(max(m * k, 1), np.int8), dev)
        b = to_dev(np.ones(max(k * n, 1), np.int8), dev)
        gk.gemm_i8(alpha, gk.MatRef(a, m, k, max(k, 1), 1), gk.MatRef(b, k, n, n, 1), beta,
                   gk.MatMut.from_row_major(cd, m, n))
        want = c0.copy()
        oracle.gemm_i8(m, k, n, alpha, np.ones(max(m * k, 1), np.int8), max(k, 1), 1,
                       np.ones(max(k * n, 1), np.int8), n, 1, beta, want, n, 1)
        assert np.array_equal(cd.cpu().numpy(), want), (alpha, beta, k)


def test_4096_cube_benchmark_shape(dev):
    """The benchmark workload, every element: against the CPU port of gemmkit's
    i8 path (oracle/cpu_port.c, itself pinned bit-exact to the oracle's closed
    form in test_oracle.py), plus sampled rows against the closed form directly
    and the exact checksum sum_i C[i, j] == sum_p (sum_i A[i, p]) B[p, j] for
    every column."""
    import torch
    M = K = N = 4096
    a = oracle.rng_i8_full(1, M * K)
    b = oracle.rng_i8_full(2, K * N)  # B column-major: element (p, j) at b[j*K + p]
    ad, bd = to_dev(a, dev), to_dev(b, dev)
    cd = torch.empty(M * N, dtype=torch.int32, device=dev)
    gk.gemm_i8(1, gk.MatRef.from_row_major(ad, M, K), gk.MatRef(bd, K, N, 1, K), 0,
               gk.MatMut.from_row_major(cd, M, N))
    got = cd.cpu().numpy()
    rows = [0, 1, 255, 256, 1023, 2048, 3071, 4095]
    for r in rows:
        want = np.zeros(N, np.int32)
        oracle.gemm_i8(1, K, N, 1, a[r * K:(r + 1) * K], K, 1, b, 1, K, 0, want, N, 1)
        assert np.array_equal(got[r * N:(r + 1) * N], want), f"row {r}"
    colsum = oracle.colsum_i32(M, N, got, N, 1)
    abft = oracle.abft_i8(M, K, N, a, K, 1, b, 1, K)
    assert np.array_equal(colsum, abft)
    full = np.empty(M * N, np.int32)
    oracle.port_gemm_i8(M, K, N, 1, a, K, 1, b, 1, K, 0, full, N, 1)
    bad = np.flatnonzero(got != full)
    assert bad.size == 0, f"{bad.size} of {M * N} elements differ, first at {bad[:5]}"


@pytest.mark.parametrize("m,k,n", [(300, 64, 200), (5, 96, 300), (300, 128, 9)])
def test_overlapping_rows(dev, m, k, n):
    """A read-only view whose rows overlap (row stride 16 < K): legal for A and
    B (only C is checked for self-aliasing, src/api.rs:236-250)."""
    import torch
    rsa, csa = 16, 1
    alen = (m - 1) * rsa + k
    a = oracle.rand_i8_100(0x3300 + m, alen)
    b = oracle.rand_i8_100(0x3400 + n, k * n)
    want = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a, rsa, csa, b, 1, k, 0, want, n, 1)
    c = torch.empty(m * n, dtype=torch.int32, device=dev)
    gk.gemm_i8(1, gk.MatRef(to_dev(a, dev), m, k, rsa, csa), gk.MatRef(to_dev(b, dev), k, n, 1, k),
               0, gk.MatMut.from_row_major(c, m, n))
    assert np.array_equal(c.cpu().numpy(), want)
