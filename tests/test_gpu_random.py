"""Seeded random sweep over the whole path: shapes drawn across every route's
boundaries (GEMV, skinny, small f32, streaming short-K, the tile kernels with
and without split K and the tail split), random strided layouts (row, column,
padded), alpha/beta, requantization and batches.  Each case is checked
against the oracle on the same buffers:

* i8 -> i32 and requantized i8/u8: bit-exact (or_gemm_i8, or_gemm_i8_requant);
* f32: relative Frobenius <= 1e-5 and the reference's 8*k*eps gate against
  the f64 product;
* bf16 -> f32: elementwise <= 1e-2 * max(|ref|, 1e-3 * max|ref|) against the
  f64 product of the bf16-rounded inputs;
* batched f32/bf16: every element bit-identical to its standalone call.

The draws are fixed by the seed, so a failure names a reproducible case.
"""
import numpy as np
import pytest
import torch

import gemmkit_amd as gk
import oracle
from helpers import bf16_tensor_from_bits, gather, layout_strides, scatter, to_dev
from test_gpu_float import F32_EPS, rel_frob
from test_gpu_requant import _run as run_requant

pytestmark = pytest.mark.gpu

EDGES = [1, 2, 3, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 191, 192, 193,
         255, 256, 257, 383, 513]
LAYOUTS = ["row", "col", "row+", "col+"]


def draw_dim(rng, hi):
    """Mostly route-boundary values, sometimes any value up to hi."""
    if rng.random() < 0.6:
        v = int(rng.choice(EDGES))
    else:
        v = int(rng.integers(1, hi + 1))
    return min(v, hi)


def cases(seed, n, m_hi=600, k_hi=700, n_hi=600):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        m, k, nn = draw_dim(rng, m_hi), draw_dim(rng, k_hi), draw_dim(rng, n_hi)
        la, lb, lc = (str(rng.choice(LAYOUTS)) for _ in range(3))
        out.append((i, m, k, nn, la, lb, lc, int(rng.integers(0, 1 << 30))))
    return out


@pytest.mark.parametrize("i,m,k,n,la,lb,lc,s", cases(0xA11, 120, m_hi=1100, k_hi=900, n_hi=1100))
def test_i8_random(dev, i, m, k, n, la, lb, lc, s):
    rng = np.random.default_rng(s)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int8)
    c0 = rng.integers(-1000, 1000, (m, n), dtype=np.int32)
    alpha, beta = int(rng.choice([1, 3, -2])), int(rng.choice([0, 1, -1, 5]))
    rsa, csa, al = layout_strides(m, k, la, 3)
    rsb, csb, bl = layout_strides(k, n, lb, 5)
    rsc, csc, cl = layout_strides(m, n, lc, 2)
    abuf, bbuf = scatter(a, rsa, csa, al), scatter(b, rsb, csb, bl)
    cbuf = scatter(c0, rsc, csc, cl, fill=-77)
    want = cbuf.copy()
    oracle.gemm_i8(m, k, n, alpha, abuf, rsa, csa, bbuf, rsb, csb, beta, want, rsc, csc)
    cd = to_dev(cbuf, dev)
    gk.gemm_i8(alpha, gk.MatRef(to_dev(abuf, dev), m, k, rsa, csa),
               gk.MatRef(to_dev(bbuf, dev), k, n, rsb, csb), beta, gk.MatMut(cd, m, n, rsc, csc))
    got = cd.cpu().numpy()
    assert np.array_equal(got, want), f"case {i}: {m}x{k}x{n} {la}/{lb}/{lc} a={alpha} b={beta}"


@pytest.mark.parametrize("i,m,k,n,la,lb,lc,s", cases(0xB22, 60))
def test_requant_random(dev, i, m, k, n, la, lb, lc, s):
    rng = np.random.default_rng(s)
    a = rng.integers(-127, 128, m * k, dtype=np.int8)
    b = rng.integers(-127, 128, k * n, dtype=np.int8)
    rsa, csa, al = layout_strides(m, k, la, 0)
    rsb, csb, bl = layout_strides(k, n, lb, 0)
    rsc, csc, cl = layout_strides(m, n, lc, 1)
    abuf = scatter(a.reshape(m, k), rsa, csa, al)
    bbuf = scatter(b.reshape(k, n), rsb, csb, bl)
    axis = int(rng.integers(0, 2))
    ch = n if axis else m
    per_tensor = rng.random() < 0.25
    scales = None if per_tensor else (1e-4 + rng.random(ch) * (1e-2 - 1e-4)).astype(np.float32)
    bias = rng.integers(-65536, 65537, ch, dtype=np.int32) if rng.random() < 0.7 else None
    u8 = bool(rng.random() < 0.4)
    zp = int(rng.integers(0, 256)) if u8 else int(rng.integers(-128, 128))
    relu = bool(rng.random() < 0.5)
    got, want = run_requant(dev, m, k, n, abuf, bbuf, rsa, csa, rsb, csb, 0.003, scales, zp, bias,
                            axis, relu, u8, rsc, csc, cl)
    assert np.array_equal(got, want), f"case {i}: {m}x{k}x{n} {la}/{lb}/{lc} axis={axis} u8={u8}"


@pytest.mark.parametrize("i,m,k,n,la,lb,lc,s", cases(0xC33, 100, m_hi=900, k_hi=900, n_hi=900))
def test_f32_random(dev, i, m, k, n, la, lb, lc, s):
    rng = np.random.default_rng(s)
    a = (rng.random((m, k)) * 2 - 1).astype(np.float32)
    b = (rng.random((k, n)) * 2 - 1).astype(np.float32)
    c0 = (rng.random((m, n)) * 2 - 1).astype(np.float32)
    alpha, beta = float(rng.choice([1.0, 0.5, -1.25])), float(rng.choice([0.0, 1.0, -0.75]))
    rsa, csa, al = layout_strides(m, k, la, 3)
    rsb, csb, bl = layout_strides(k, n, lb, 3)
    rsc, csc, cl = layout_strides(m, n, lc, 3)
    abuf, bbuf, cbuf = scatter(a, rsa, csa, al), scatter(b, rsb, csb, bl), scatter(c0, rsc, csc, cl)
    ref = oracle.gemm_f64(m, k, n, alpha, abuf, rsa, csa, bbuf, rsb, csb, beta, cbuf, rsc, csc)
    cd = to_dev(cbuf, dev)
    gk.gemm(alpha, gk.MatRef(to_dev(abuf, dev), m, k, rsa, csa),
            gk.MatRef(to_dev(bbuf, dev), k, n, rsb, csb), beta, gk.MatMut(cd, m, n, rsc, csc))
    got = gather(cd.cpu().numpy(), m, n, rsc, csc).astype(np.float64)
    tag = f"case {i}: {m}x{k}x{n} {la}/{lb}/{lc}"
    if np.linalg.norm(ref) > 0:
        assert rel_frob(got, ref) <= 1e-5, tag
    num = np.linalg.norm((got - ref).ravel())
    den = np.linalg.norm(a.ravel()) * np.linalg.norm(b.ravel()) * abs(alpha) + \
        abs(beta) * np.linalg.norm(c0.ravel()) + 1e-30
    assert num / den <= 8 * k * F32_EPS, tag


@pytest.mark.parametrize("i,m,k,n,la,lb,lc,s", cases(0xD44, 60, k_hi=600))
def test_bf16_f32out_random(dev, i, m, k, n, la, lb, lc, s):
    rng = np.random.default_rng(s)
    abits = oracle.bf16_bits(rng.standard_normal(m * k).astype(np.float32))
    bbits = oracle.bf16_bits(rng.standard_normal(k * n).astype(np.float32))
    af, bf = oracle.bf16_to_f32(abits).reshape(m, k), oracle.bf16_to_f32(bbits).reshape(k, n)
    rsa, csa, al = layout_strides(m, k, la, 8)
    rsb, csb, bl = layout_strides(k, n, lb, 8)
    abuf = scatter(abits.reshape(m, k), rsa, csa, al)
    bbuf = scatter(bbits.reshape(k, n), rsb, csb, bl)
    alpha = float(rng.choice([1.0, 1 / np.sqrt(128.0)]))
    ref = oracle.gemm_f64(m, k, n, alpha, af.ravel(), k, 1, bf.ravel(), n, 1)
    c = torch.empty(m * n, dtype=torch.float32, device=dev)
    gk.gemm_bf16_f32out(alpha, gk.MatRef(bf16_tensor_from_bits(abuf, dev), m, k, rsa, csa),
                        gk.MatRef(bf16_tensor_from_bits(bbuf, dev), k, n, rsb, csb), 0.0,
                        gk.MatMut.from_row_major(c, m, n))
    got = c.cpu().numpy().reshape(m, n).astype(np.float64)
    floor = 1e-3 * np.abs(ref).max()
    ok = np.abs(got - ref) <= 1e-2 * np.maximum(np.abs(ref), floor)
    assert ok.all(), f"case {i}: {m}x{k}x{n} {la}/{lb}: {np.count_nonzero(~ok)} elements off"


@pytest.mark.parametrize("i,m,k,n,la,lb,lc,s", cases(0xE55, 20, m_hi=300, k_hi=400, n_hi=300))
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_batched_random(dev, i, m, k, n, la, lb, lc, s, dt):
    rng = np.random.default_rng(s)
    batch = int(rng.integers(2, 6))
    g = torch.Generator().manual_seed(s)
    a = torch.randn(batch * m * k, generator=g).to(dt).to(dev)
    b = torch.randn(batch * k * n, generator=g).to(dt).to(dev)
    out_dt = torch.float32
    c = torch.zeros(batch * m * n, dtype=out_dt, device=dev)
    rsa, csa, _ = layout_strides(m, k, la.rstrip("+"), 0)
    rsb, csb, _ = layout_strides(k, n, lb.rstrip("+"), 0)
    if dt == torch.float32:
        gk.gemm_batched_unchecked(batch, m, k, n, 1.0, a, rsa, csa, m * k, b, rsb, csb, k * n, 0.0,
                                  c, n, 1, m * n)
    else:
        gk.gemm_batched_bf16_f32out(batch, 1.0, gk.MatRef(a, m, k, rsa, csa), m * k,
                                    gk.MatRef(b, k, n, rsb, csb), k * n, 0.0,
                                    gk.MatMut.from_row_major(c, m, n), m * n)
    for z in range(batch):
        one = torch.zeros(m * n, dtype=out_dt, device=dev)
        az, bz = a[z * m * k:(z + 1) * m * k], b[z * k * n:(z + 1) * k * n]
        if dt == torch.float32:
            gk.gemm(1.0, gk.MatRef(az, m, k, rsa, csa), gk.MatRef(bz, k, n, rsb, csb), 0.0,
                    gk.MatMut.from_row_major(one, m, n))
        else:
            gk.gemm_bf16_f32out(1.0, gk.MatRef(az, m, k, rsa, csa), gk.MatRef(bz, k, n, rsb, csb),
                                0.0, gk.MatMut.from_row_major(one, m, n))
        assert torch.equal(c[z * m * n:(z + 1) * m * n], one), f"case {i} element {z}"


def large_cases(seed, n):
    """Big-tile shapes: sides across the 256-tile and one-round boundaries
    (the 16x16-MFMA tile, the 352/384-wide one-round plans, the tail split),
    K across the 128-byte stage edges."""
    rng = np.random.default_rng(seed)
    sides = [1024, 2047, 2048, 2049, 2816, 3000, 4096, 4100]
    ks = [128, 200, 1000, 2048, 4096, 4100]
    out = []
    for i in range(n):
        m = int(rng.choice(sides)) if rng.random() < 0.6 else int(rng.integers(1000, 4200))
        nn = int(rng.choice(sides)) if rng.random() < 0.6 else int(rng.integers(1000, 4200))
        k = int(rng.choice(ks)) if rng.random() < 0.6 else int(rng.integers(128, 4200))
        la, lb, lc = (str(rng.choice(LAYOUTS)) for _ in range(3))
        out.append((i, m, k, nn, la, lb, lc, int(rng.integers(0, 1 << 30))))
    return out


@pytest.mark.parametrize("i,m,k,n,la,lb,lc,s", large_cases(0xF66, 10))
def test_i8_large_random(dev, i, m, k, n, la, lb, lc, s):
    """Every element against the CPU port of gemmkit's i8 path (pinned
    bit-exact to the oracle's closed form in test_oracle.py)."""
    rng = np.random.default_rng(s)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (k, n), dtype=np.int8)
    c0 = rng.integers(-1000, 1000, (m, n), dtype=np.int32)
    alpha, beta = int(rng.choice([1, 3, -2])), int(rng.choice([0, 1, -1]))
    rsa, csa, al = layout_strides(m, k, la, 16)
    rsb, csb, bl = layout_strides(k, n, lb, 16)
    rsc, csc, cl = layout_strides(m, n, lc, 4)
    abuf, bbuf = scatter(a, rsa, csa, al), scatter(b, rsb, csb, bl)
    cbuf = scatter(c0, rsc, csc, cl, fill=-77)
    want = cbuf.copy()
    oracle.port_gemm_i8(m, k, n, alpha, abuf, rsa, csa, bbuf, rsb, csb, beta, want, rsc, csc)
    cd = to_dev(cbuf, dev)
    gk.gemm_i8(alpha, gk.MatRef(to_dev(abuf, dev), m, k, rsa, csa),
               gk.MatRef(to_dev(bbuf, dev), k, n, rsb, csb), beta, gk.MatMut(cd, m, n, rsc, csc))
    got = cd.cpu().numpy()
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"case {i}: {m}x{k}x{n} {la}/{lb}/{lc}: {bad.size} elements differ"


@pytest.mark.parametrize("i,m,k,n,la,lb,lc,s", large_cases(0xF77, 6))
def test_requant_large_random(dev, i, m, k, n, la, lb, lc, s):
    """Requantized big-tile products, every byte against the CPU port's
    requantizing path."""
    import torch
    rng = np.random.default_rng(s)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (k, n), dtype=np.int8)
    rsa, csa, al = layout_strides(m, k, la, 16)
    rsb, csb, bl = layout_strides(k, n, lb, 16)
    rsc, csc, cl = layout_strides(m, n, lc, 4)
    abuf, bbuf = scatter(a, rsa, csa, al), scatter(b, rsb, csb, bl)
    axis = int(rng.integers(0, 2))
    ch = n if axis else m
    scales = (1e-4 + rng.random(ch) * (1e-2 - 1e-4)).astype(np.float32)
    bias = rng.integers(-65536, 65537, ch, dtype=np.int32)
    u8 = bool(rng.random() < 0.4)
    zp = int(rng.integers(0, 256)) if u8 else int(rng.integers(-128, 128))
    relu = bool(rng.random() < 0.5)
    lo, hi = (0, 255) if u8 else (-128, 127)
    lo_eff = max(lo, zp) if relu else lo
    want = np.zeros(cl, np.uint8)
    oracle.port_gemm_i8_requant(m, k, n, abuf, rsa, csa, bbuf, rsb, csb, 0.0, scales, zp, bias,
                                axis, lo_eff, hi, want, rsc, csc)
    cd = torch.zeros(cl, dtype=torch.uint8 if u8 else torch.int8, device=dev)
    sd = to_dev(scales, dev)
    req = gk.Requantize(gk.RequantScale.PerCol(sd) if axis else gk.RequantScale.PerRow(sd), zp,
                        to_dev(bias, dev), bias_axis="col" if axis else "row", relu=relu)
    (gk.gemm_i8_requant_u8 if u8 else gk.gemm_i8_requant)(
        gk.MatRef(to_dev(abuf, dev), m, k, rsa, csa), gk.MatRef(to_dev(bbuf, dev), k, n, rsb, csb),
        req, gk.MatMut(cd, m, n, rsc, csc))
    got = cd.cpu().numpy().view(np.uint8)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"case {i}: {m}x{k}x{n} {la}/{lb}/{lc} axis={axis} u8={u8}: {bad.size} differ"


@pytest.mark.parametrize("i,m,k,n,la,lb,lc,s", large_cases(0xF88, 4))
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_bf16_large_random(dev, i, m, k, n, la, lb, lc, s, out):
    """Big-tile bf16 products (the 16x16-MFMA tile and the one-round plans)
    against the f64 product of the bf16-rounded inputs (numpy's f64 matmul: the
    closed form at this size), elementwise within the bf16 bar."""
    rng = np.random.default_rng(s)
    abits = oracle.bf16_bits(rng.standard_normal(m * k).astype(np.float32))
    bbits = oracle.bf16_bits(rng.standard_normal(k * n).astype(np.float32))
    af = oracle.bf16_to_f32(abits).reshape(m, k).astype(np.float64)
    bf = oracle.bf16_to_f32(bbits).reshape(k, n).astype(np.float64)
    rsa, csa, al = layout_strides(m, k, la, 8)
    rsb, csb, bl = layout_strides(k, n, lb, 8)
    abuf = scatter(abits.reshape(m, k), rsa, csa, al)
    bbuf = scatter(bbits.reshape(k, n), rsb, csb, bl)
    ref = af @ bf
    A = gk.MatRef(bf16_tensor_from_bits(abuf, dev), m, k, rsa, csa)
    B = gk.MatRef(bf16_tensor_from_bits(bbuf, dev), k, n, rsb, csb)
    if out == "f32":
        c = torch.empty(m * n, dtype=torch.float32, device=dev)
        gk.gemm_bf16_f32out(1.0, A, B, 0.0, gk.MatMut.from_row_major(c, m, n))
    else:
        c = torch.empty(m * n, dtype=torch.bfloat16, device=dev)
        gk.gemm(1.0, A, B, 0.0, gk.MatMut.from_row_major(c, m, n))
    got = c.float().cpu().numpy().reshape(m, n).astype(np.float64)
    floor = 1e-3 * np.abs(ref).max()
    ok = np.abs(got - ref) <= 1e-2 * np.maximum(np.abs(ref), floor)
    assert ok.all(), f"case {i}: {m}x{k}x{n} {la}/{lb} {out}: {np.count_nonzero(~ok)} elements off"
