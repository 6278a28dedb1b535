"""GPU parity: requantizing i8 GEMM (i8 and u8 output) against the oracle, bit-exact.

Covers the reference's own requant tests (tests/epilogue/requant.rs): the
round-half-even ties KAT (:253-272), vector ties at m = 37, zp = 3 (:449-480),
extreme accumulators and i32-extreme biases (:486-545), the k == 0 fill
(:548-575), the per-row scale pattern (:1211-1219), the u8 twin, plus this
engine's per-column and ReLU extensions and the int8 linear layer
(2048 x 4096 x 11008, prepacked weights) at full size.
"""
import numpy as np
import pytest

import gemmkit_amd as gk
import oracle
from helpers import layout_strides, scatter, to_dev

pytestmark = pytest.mark.gpu


def _run(dev, m, k, n, a, b, rsa, csa, rsb, csb, scale, scales, zp, bias, axis, relu, u8,
         rsc, csc, clen, packed=False):
    """Runs the GPU requant GEMM and the oracle on the same buffers; returns both."""
    import torch
    lo, hi = (0, 255) if u8 else (-128, 127)
    lo_eff = max(lo, zp) if relu else lo
    want = np.zeros(clen, np.uint8 if u8 else np.int8)
    oracle.gemm_i8_requant(m, k, n, a, rsa, csa, b, rsb, csb, scale, scales, zp, bias, axis,
                           lo_eff, hi, want, rsc, csc)
    ad, bd = to_dev(a, dev), to_dev(b, dev)
    cd = torch.zeros(clen, dtype=torch.uint8 if u8 else torch.int8, device=dev)
    if scales is None:
        sc = gk.RequantScale.PerTensor(scale)
    elif axis == 0:
        sc = gk.RequantScale.PerRow(to_dev(np.asarray(scales, np.float32), dev))
    else:
        sc = gk.RequantScale.PerCol(to_dev(np.asarray(scales, np.float32), dev))
    bt = None if bias is None else to_dev(np.asarray(bias, np.int32), dev)
    req = gk.Requantize(sc, zp, bt, bias_axis="col" if axis else "row", relu=relu)
    av = gk.MatRef(ad, m, k, rsa, csa)
    cv = gk.MatMut(cd, m, n, rsc, csc)
    if packed:
        p = gk.prepack_rhs_i8(gk.MatRef(bd, k, n, rsb, csb))
        (gk.gemm_i8_packed_b_requant_u8 if u8 else gk.gemm_i8_packed_b_requant)(av, p, req, cv)
    else:
        (gk.gemm_i8_requant_u8 if u8 else gk.gemm_i8_requant)(av, gk.MatRef(bd, k, n, rsb, csb),
                                                              req, cv)
    return cd.cpu().numpy(), want


def test_ties_even_exact(dev):
    # tests/epilogue/requant.rs:253-272, expected values from the reference test
    a = np.array([1, 3, 5, 7, -1, -3], np.int8)
    b = np.array([1], np.int8)
    got, want = _run(dev, 6, 1, 1, a, b, 1, 6, 1, 1, 0.5, None, 0, None, 0, False, False,
                     1, 6, 6)
    assert list(got) == [0, 2, 2, 4, 0, -2]
    assert list(want) == [0, 2, 2, 4, 0, -2]


def test_vector_ties_zp3(dev):
    # tests/epilogue/requant.rs:449-480
    m = 37
    a = np.array([i - 18 for i in range(m)], np.int8)
    b = np.array([1], np.int8)
    got, want = _run(dev, m, 1, 1, a, b, 1, m, 1, 1, 0.5, None, 3, None, 0, False, False,
                     1, m, m)
    expect = [oracle.requant_one(int(v), 0, 0.5, 3) for v in a]
    assert np.array_equal(got, want)
    assert list(got) == expect


@pytest.mark.parametrize("scale", [1.0, 1e-9, 0.5, 1e30])
@pytest.mark.parametrize("zp", [0, -128, 127])
@pytest.mark.parametrize("u8", [False, True])
def test_extreme_accumulators(dev, scale, zp, u8):
    # tests/epilogue/requant.rs:486-545: a, b in {-128, 127}, bias at the i32 extremes
    m, k, n = 37, 1, 7
    a = np.array([-128 if i % 2 == 0 else 127 for i in range(m * k)], np.int8)
    b = np.array([127 if j % 2 == 0 else -128 for j in range(k * n)], np.int8)
    bias = np.array([[2**31 - 1, -2**31, 2**31 - 1 - 200, -2**31 + 200][i % 4] for i in range(m)],
                    np.int32)
    zp_eff = zp if not u8 else max(zp, 0)
    for rsc, csc, clen in [(1, m, m * n), (2, 2 * m, 2 * m * n)]:
        got, want = _run(dev, m, k, n, a, b, 1, m, 1, k, scale, None, zp_eff, bias, 0, False, u8,
                         rsc, csc, clen)
        assert np.array_equal(got, want), (scale, zp, rsc)


def test_degenerate_k0(dev):
    # tests/epilogue/requant.rs:548-575
    m, n = 12, 10
    bias = np.array([i * 40 - 200 for i in range(m)], np.int32)
    a = np.zeros(1, np.int8)
    b = np.zeros(1, np.int8)
    got, want = _run(dev, m, 0, n, a, b, 1, m, 1, 0, 0.5, None, 7, bias, 0, False, False,
                     1, m, m * n)
    assert np.array_equal(got, want)
    expect = np.array([[oracle.requant_one(0, int(bias[i]), 0.5, 7) for i in range(m)]
                       for _ in range(n)], np.int8).ravel()
    assert np.array_equal(got, expect)


PER_ROW_PATTERN = [0.003, 0.5, 1.0, 7.25, 0.0078125, 0.1]


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 13, 5), (37, 300, 9), (64, 1000, 70),
                                   (130, 512, 260), (300, 777, 333), (512, 2048, 384)])
@pytest.mark.parametrize("row_major_c", [False, True])
@pytest.mark.parametrize("u8", [False, True])
def test_per_row_scale_bias(dev, m, k, n, row_major_c, u8):
    # tests/epilogue/requant.rs:1195-1260 shape of test: per-row scales, bias in
    # [-1000, 1000], A and B column-major, both C orientations
    rng = oracle.rng_i8_sym127
    a = rng(m * 7 + k, m * k)
    b = rng(n * 3 + k, k * n)
    bias = (oracle.rng_next_u64(99 + m, m) if m else [])
    bias = np.array([(v % 2001) - 1000 for v in bias], np.int32)
    scales = np.array([PER_ROW_PATTERN[i % 6] for i in range(m)], np.float32)
    rsc, csc = (n, 1) if row_major_c else (1, m)
    zp = 5 if u8 else -3
    got, want = _run(dev, m, k, n, a, b, 1, m, 1, k, 0.0, scales, zp, bias, 0, False, u8,
                     rsc, csc, m * n)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("m,k,n", [(5, 64, 3), (96, 256, 200), (257, 1024, 511)])
@pytest.mark.parametrize("la,lb,lc", [("row", "col", "row"), ("col", "row", "col"),
                                      ("row+", "row+", "col+")])
@pytest.mark.parametrize("per", ["tensor", "col"])
@pytest.mark.parametrize("relu", [False, True])
def test_extensions_per_col_relu(dev, m, k, n, la, lb, lc, per, relu):
    a = oracle.rng_i8_sym127(1000 + m, m * k).reshape(m, k)
    b = oracle.rng_i8_sym127(2000 + n, k * n).reshape(k, n)
    rsa, csa, al = layout_strides(m, k, la, 5)
    rsb, csb, bl = layout_strides(k, n, lb, 5)
    rsc, csc, cl = layout_strides(m, n, lc, 5)
    abuf, bbuf = scatter(a, rsa, csa, al), scatter(b, rsb, csb, bl)
    u = oracle.rng_unit(77 + n, 2 * n)
    scales = (1e-4 + (u[:n] + 1) / 2 * (1e-2 - 1e-4)).astype(np.float32)
    bias = np.round(u[n:] * 65536).astype(np.int32)
    if per == "tensor":
        got, want = _run(dev, m, k, n, abuf, bbuf, rsa, csa, rsb, csb, 0.004, None, 0, None, 0,
                         relu, False, rsc, csc, cl)
    else:
        got, want = _run(dev, m, k, n, abuf, bbuf, rsa, csa, rsb, csb, 0.0, scales, 0, bias, 1,
                         relu, False, rsc, csc, cl)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("u8", [False, True])
def test_packed_requant_matches_plain(dev, u8):
    m, k, n = 200, 4096, 300
    a = oracle.rng_i8_sym127(5, m * k)
    b = oracle.rng_i8_sym127(6, n * k)   # B column-major (k x n): W rows
    u = oracle.rng_unit(7, 2 * n)
    scales = (1e-4 + (u[:n] + 1) / 2 * (1e-2 - 1e-4)).astype(np.float32)
    bias = np.round(u[n:] * 65536).astype(np.int32)
    zp = 17 if u8 else 0
    got, want = _run(dev, m, k, n, a, b, k, 1, 1, k, 0.0, scales, zp, bias, 1, True, u8,
                     n, 1, m * n, packed=True)
    assert np.array_equal(got, want)


def test_linear_layer_full_size(dev):
    """The int8 linear layer at full size: Y (2048 x 11008, token-major) =
    requant(X (2048 x 4096) . W^T), W prepacked once and reused, per-output-channel
    scale and bias, zp 0, ReLU.  Every element is checked against the CPU port
    of gemmkit's paths (oracle/cpu_port.c, pinned bit-exact to the oracle's
    closed forms in test_oracle.py): the i32 GEMM of the same operands against
    the port's i32 GEMM (and sampled rows against the closed form, plus the
    exact column checksum), and the fused bytes, on two calls, against the
    port's requantizing path on a prepacked W and against the oracle's requant
    map of the port's i32."""
    import torch
    T, K, Nc = 2048, 4096, 11008
    x = oracle.rng_i8_sym127(21, T * K)
    w = oracle.rng_i8_sym127(22, Nc * K)
    u = oracle.rng_unit(23, 2 * Nc)
    bias = np.round(u[:Nc] * 65536).astype(np.int32)
    scale = (1e-4 + (u[Nc:] + 1) / 2 * (1e-2 - 1e-4)).astype(np.float32)
    xd, wd = to_dev(x, dev), to_dev(w, dev)
    acc = torch.empty(T * Nc, dtype=torch.int32, device=dev)
    gk.gemm_i8(1, gk.MatRef.from_row_major(xd, T, K), gk.MatRef(wd, K, Nc, 1, K), 0,
               gk.MatMut.from_row_major(acc, T, Nc))
    acc_h = acc.cpu().numpy()
    del acc
    for r in (0, 777, 2047):
        row = np.zeros(Nc, np.int32)
        oracle.gemm_i8(1, K, Nc, 1, x[r * K:(r + 1) * K], K, 1, w, 1, K, 0, row, Nc, 1)
        assert np.array_equal(acc_h[r * Nc:(r + 1) * Nc], row), f"row {r}"
    assert np.array_equal(oracle.colsum_i32(T, Nc, acc_h, Nc, 1),
                          oracle.abft_i8(T, K, Nc, x, K, 1, w, 1, K))
    acc_port = np.empty(T * Nc, np.int32)
    oracle.port_gemm_i8(T, K, Nc, 1, x, K, 1, w, 1, K, 0, acc_port, Nc, 1)
    assert np.array_equal(acc_h, acc_port)
    want = np.zeros(T * Nc, np.int8)
    oracle.requant_map(T, Nc, acc_port, Nc, 1, 0.0, scale, 0, bias, 1, 0, 127, want, Nc, 1)
    want_port = np.zeros(T * Nc, np.int8)
    pb = oracle.PortPackedB(K, Nc, w, 1, K)
    oracle.port_gemm_i8_requant(T, K, Nc, x, K, 1, None, 0, 0, 0.0, scale, 0, bias, 1, 0, 127,
                                want_port.view(np.uint8), Nc, 1, packed=pb)
    assert np.array_equal(want_port, want)
    packed = gk.prepack_rhs_i8(gk.MatRef(wd, K, Nc, 1, K))
    req = gk.Requantize(gk.RequantScale.PerCol(to_dev(scale, dev)), 0, to_dev(bias, dev),
                        bias_axis="col", relu=True)
    y = torch.empty(T * Nc, dtype=torch.int8, device=dev)
    for _ in range(2):
        y.fill_(99)
        gk.gemm_i8_packed_b_requant(gk.MatRef.from_row_major(xd, T, K), packed, req,
                                    gk.MatMut.from_row_major(y, T, Nc))
        got = y.cpu().numpy()
        assert np.array_equal(got, want)
    # the outputs mix saturated and in-range values
    assert (got == 127).any() and ((got > 0) & (got < 127)).any() and (got == 0).any()
