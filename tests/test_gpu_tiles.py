"""GPU parity of every matrix-core tile, each forced with GEMMKIT_HIP_TILE
(which also turns off split K, the tail split and the streaming kernel), on
ragged shapes: i8 with alpha/beta and requantized outputs bit-exact against
the oracle; bf16 and f32 outputs identical across all 32x32-MFMA tiles (every
one feeds each output's K chunks to the matrix cores in the same order) and
within the float bars against the f64 product; the 16x16-MFMA tile (bf16
only: it sums 32 k per instruction) within the same bars.  The 16x16-MFMA
strip tile (256 x 352) takes int8 inputs only."""
import os

import numpy as np
import pytest
import torch

import gemmkit_amd as gk
import oracle
from helpers import to_dev

pytestmark = pytest.mark.gpu

TILES = sorted(gk.TILE_NAMES.values())
M16 = "256x256w8m16"  # 16x16 MFMAs: int8 and bf16 inputs only
I8_ONLY = {"256x352w8m16"}  # the 16x16-MFMA strip tile: int8 inputs only
TILES_F = [t for t in TILES if t not in I8_ONLY]


class tile:
    def __init__(self, name):
        self.name = name

    def __enter__(self):
        self.old = os.environ.get("GEMMKIT_HIP_TILE")
        os.environ["GEMMKIT_HIP_TILE"] = self.name

    def __exit__(self, *exc):
        if self.old is None:
            del os.environ["GEMMKIT_HIP_TILE"]
        else:
            os.environ["GEMMKIT_HIP_TILE"] = self.old


@pytest.mark.parametrize("name", TILES)
@pytest.mark.parametrize("m,k,n", [(300, 520, 200), (129, 64, 1000), (517, 1040, 389)])
def test_i8_every_tile(dev, name, m, k, n):
    a = oracle.rng_i8_full(0x701 + m, m * k)
    b = oracle.rng_i8_full(0x702 + n, k * n)  # B column-major
    c0 = ((np.arange(m * n) % 11) - 5).astype(np.int32)
    want = c0.copy()
    oracle.gemm_i8(m, k, n, 3, a, k, 1, b, 1, k, -2, want, n, 1)
    c = to_dev(c0, dev)
    with tile(name):
        gk.gemm_i8(3, gk.MatRef.from_row_major(to_dev(a, dev), m, k),
                   gk.MatRef(to_dev(b, dev), k, n, 1, k), -2, gk.MatMut.from_row_major(c, m, n))
    assert np.array_equal(c.cpu().numpy(), want)


@pytest.mark.parametrize("name", TILES)
@pytest.mark.parametrize("axis", [0, 1])
def test_requant_every_tile(dev, name, axis):
    m, k, n = 333, 1024, 421
    a = oracle.rng_i8_sym127(0x711, m * k)
    b = oracle.rng_i8_sym127(0x712, k * n)
    ch = n if axis else m
    u = oracle.rng_unit(0x713 + ch, 2 * ch)
    scales = (1e-4 + (u[:ch] + 1) / 2 * (1e-2 - 1e-4)).astype(np.float32)
    bias = np.round(u[ch:] * 65536).astype(np.int32)
    acc = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a, k, 1, b, 1, k, 0, acc, n, 1)
    want = np.zeros(m * n, np.uint8)
    oracle.requant_map(m, n, acc, n, 1, 0.0, scales, -3, bias, axis, -128, 127, want, n, 1)
    sd, bd = to_dev(scales, dev), to_dev(bias, dev)
    req = gk.Requantize(gk.RequantScale.PerCol(sd) if axis else gk.RequantScale.PerRow(sd),
                        zero_point=-3, bias=bd, bias_axis="col" if axis else "row")
    c = torch.zeros(m * n, dtype=torch.int8, device=dev)
    with tile(name):
        gk.gemm_i8_requant(gk.MatRef.from_row_major(to_dev(a, dev), m, k),
                           gk.MatRef(to_dev(b, dev), k, n, 1, k), req,
                           gk.MatMut.from_row_major(c, m, n))
    assert np.array_equal(c.cpu().numpy().view(np.uint8), want)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_float_tiles_identical(dev, dt):
    m, k, n = 300, 272, 410
    g = torch.Generator().manual_seed(21)
    a = torch.randn(m * k, generator=g).to(dt).to(dev)
    b = torch.randn(k * n, generator=g).to(dt).to(dev)
    c0 = torch.randn(m * n, generator=g).to(dev)
    outs = {}
    for name in TILES_F:
        if name == M16 and dt == torch.float32:
            continue
        c = c0.clone()
        with tile(name):
            if dt == torch.bfloat16:
                gk.gemm_bf16_f32out(0.5, gk.MatRef.from_row_major(a, m, k),
                                    gk.MatRef(b, k, n, 1, k), 1.0, gk.MatMut.from_row_major(c, m, n))
            else:
                gk.gemm(0.5, gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k), 1.0,
                        gk.MatMut.from_row_major(c, m, n))
        outs[name] = c
    same = [t for t in TILES_F if t != M16]
    first = outs[same[0]]
    for name in same[1:]:
        assert torch.equal(outs[name], first), name
    ref = 0.5 * (a.double().cpu().reshape(m, k) @ b.double().cpu().reshape(n, k).T) + \
        c0.double().cpu().reshape(m, n)
    for name in [same[0]] + ([M16] if M16 in outs else []):
        err = (outs[name].double().cpu().reshape(m, n) - ref).norm() / ref.norm()
        assert err <= (1e-5 if dt == torch.float32 else 1e-2), name


@pytest.mark.parametrize("name", TILES_F)
def test_batched_bf16_every_tile(dev, name):
    """Each element of a batched bf16 product (grid z, B shared through a zero
    batch stride, C element stride past its extent) equals its standalone
    call on the same forced tile, bit for bit, with f32 and bf16 output."""
    batch, m, k, n = 3, 270, 320, 300
    g = torch.Generator().manual_seed(0x7B1)
    a = torch.randn(batch * m * k, generator=g).to(torch.bfloat16).to(dev)
    b = torch.randn(k * n, generator=g).to(torch.bfloat16).to(dev)
    cbs = m * n + 64
    for out in (torch.float32, torch.bfloat16):
        c = torch.zeros(batch * cbs, dtype=out, device=dev)
        with tile(name):
            if out == torch.float32:
                gk.gemm_batched_bf16_f32out(batch, 0.75, gk.MatRef.from_row_major(a, m, k), m * k,
                                            gk.MatRef(b, k, n, 1, k), 0, 0.0,
                                            gk.MatMut.from_row_major(c, m, n), cbs)
            else:
                gk.gemm_batched(batch, 0.75, gk.MatRef.from_row_major(a, m, k), m * k,
                                gk.MatRef(b, k, n, 1, k), 0, 0.0,
                                gk.MatMut.from_row_major(c, m, n), cbs)
            for z in range(batch):
                s = torch.zeros(m * n, dtype=out, device=dev)
                az = a[z * m * k:(z + 1) * m * k]
                if out == torch.float32:
                    gk.gemm_bf16_f32out(0.75, gk.MatRef.from_row_major(az, m, k),
                                        gk.MatRef(b, k, n, 1, k), 0.0,
                                        gk.MatMut.from_row_major(s, m, n))
                else:
                    gk.gemm(0.75, gk.MatRef.from_row_major(az, m, k), gk.MatRef(b, k, n, 1, k),
                            0.0, gk.MatMut.from_row_major(s, m, n))
                got = c[z * cbs:z * cbs + m * n]
                assert torch.equal(got.view(torch.int16) if out == torch.bfloat16 else got,
                                   s.view(torch.int16) if out == torch.bfloat16 else s), (name, z)
                assert (c[z * cbs + m * n:(z + 1) * cbs] == 0).all()


EDGE_TILES = [M16, "256x352w8m16", "128x128"]


@pytest.mark.parametrize("name", EDGE_TILES)
@pytest.mark.parametrize("case", ["ties", "onehalf", "big", "nonfinite", "u8relu", "i8relu", "tensor"])
@pytest.mark.parametrize("axis", [0, 1])
def test_requant_edges_every_16x16_tile(dev, name, case, axis):
    """The requantizing store's tiers through the 16x16-MFMA tiles (a 32x32
    tile as the control), bit-exact against the oracle: products on a half
    (scale 1/2 on odd accumulators, for every channel or for one), operands beyond 2^24 (biases near the
    i32 edges), non-finite and huge channel scales (unchecked entry: inf, NaN,
    3e38), u8 and i8 output with ReLU, a per-tensor scale.  C's row stride (424) is a
    multiple of 4 while n = 421 is not, so whole chunks take the vector store
    and the last chunk of each row the element-wise one."""
    m, k, n, ldc = 333, 1024, 421, 424
    a = oracle.rng_i8_sym127(0x721, m * k)
    b = oracle.rng_i8_sym127(0x722, k * n)
    ch = n if axis else m
    u = oracle.rng_unit(0x723 + ch, 2 * ch)
    scales = (1e-4 + (u[:ch] + 1) / 2 * (1e-2 - 1e-4)).astype(np.float32)
    bias = np.round(u[ch:] * 65536).astype(np.int32)
    zp, u8, relu, scale = -3, False, False, 0.0
    if case == "ties":
        scales[:] = 0.5
        bias[::2] += 1
    elif case == "onehalf":  # one channel on halves: single chunks of a row block need the tie tier
        scales[37] = 0.5
    elif case == "big":
        bias[::3] = 2**31 - 1 - np.arange(0, ch, 3, dtype=np.int64) % 1000
        bias[1::3] = -2**31 + np.arange(1, ch, 3, dtype=np.int64) % 1000
        scales[::5] = 1e-9
    elif case == "nonfinite":
        scales[7] = np.inf
        scales[100] = np.nan
        scales[200] = 3e38
    elif case == "u8relu":
        zp, u8, relu = 5, True, True
    elif case == "i8relu":  # the band [3, 127] starts above zero
        zp, relu = 3, True
    else:
        scale, scales = 0.5, None
    lo, hi = (0, 255) if u8 else (-128, 127)
    acc = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a, k, 1, b, 1, k, 0, acc, n, 1)
    want = np.full(m * ldc, 0x5A, np.uint8)
    oracle.requant_map(m, n, acc, n, 1, scale, scales, zp, bias, axis,
                       max(lo, zp) if relu else lo, hi, want, ldc, 1)
    c = torch.full((m * ldc,), 0x5A, dtype=torch.uint8, device=dev)
    fn = gk.gemm_i8_requant_u8_unchecked if u8 else gk.gemm_i8_requant_unchecked
    with tile(name):
        fn(m, k, n, to_dev(a, dev), k, 1, to_dev(b, dev), 1, k, scale,
           None if scales is None else to_dev(scales, dev), zp, to_dev(bias, dev), c, ldc, 1,
           axis=axis, relu=relu)
    assert np.array_equal(c.cpu().numpy(), want), (name, case, axis)


@pytest.mark.parametrize("name", [M16, "256x352w8m16"])
@pytest.mark.parametrize("alpha,beta", [(1, 0), (1, 1), (-1, 0), (2, -3)])
def test_i8_stepped_stores_16x16_tiles(dev, name, alpha, beta):
    """The 16x16-MFMA tiles' stepped-address i32 stores (alpha = 1 without
    multiplies) with a padded row stride: whole chunks vector-stored, the
    ragged last chunk element-wise, the padding untouched."""
    m, k, n, ldc = 517, 640, 389, 392
    a = oracle.rng_i8_full(0x731, m * k)
    b = oracle.rng_i8_full(0x732, k * n)
    c0 = ((np.arange(m * ldc) % 13) - 6).astype(np.int32)
    want = c0.copy()
    oracle.gemm_i8(m, k, n, alpha, a, k, 1, b, 1, k, beta, want, ldc, 1)
    c = to_dev(c0, dev)
    with tile(name):
        gk.gemm_i8(alpha, gk.MatRef.from_row_major(to_dev(a, dev), m, k),
                   gk.MatRef(to_dev(b, dev), k, n, 1, k), beta, gk.MatMut(c, m, n, ldc, 1))
    assert np.array_equal(c.cpu().numpy(), want)


@pytest.mark.parametrize("m,k,n,layout", [(333, 1024, 421, "row424"), (257, 512, 259, "row"),
                                          (300, 640, 270, "col"), (256, 256, 256, "row")])
def test_bf16_f32out_exact_16x16_tile(dev, m, k, n, layout):
    """The 16x16-MFMA tile's f32 output (unfused: restaged as whole tile rows
    and written through the L2) on integer-valued bf16 operands, where every
    product, sum, alpha*acc + beta*C and the f32 result are exact: equal bit
    for bit to the int64 product.  Covers a row stride that is a multiple of 4
    with n not (whole chunks by vector, the last chunk element-wise), a row
    stride that is not (element-wise), a column-major C (taken as the
    transposed product) and a tile-aligned shape; the bytes around C stay."""
    g = torch.Generator().manual_seed(0x7C1 + m)
    ai = torch.randint(-8, 9, (m * k,), generator=g)
    bi = torch.randint(-8, 9, (k * n,), generator=g)  # B column-major: (p, j) at j*k + p
    c0 = torch.randint(-64, 65, (m * n,), generator=g).double() / 4
    want = (0.75 * (ai.reshape(m, k).double() @ bi.reshape(n, k).double().T) +
            0.5 * c0.reshape(m, n))  # |values| < 2^24 * 0.25: exact in f32
    if layout == "col":
        ld = m
        cfull = torch.full((n * ld + 32,), -7.0, dtype=torch.float32)
        cfull[:n * ld] = c0.reshape(m, n).T.contiguous().reshape(-1).float()
        cm = lambda t: gk.MatMut(t, m, n, 1, ld)  # noqa: E731
        got_of = lambda t: t[:n * ld].reshape(n, ld)[:, :m].T  # noqa: E731
    else:
        ld = 424 if layout == "row424" else n
        cfull = torch.full((m * ld + 32,), -7.0, dtype=torch.float32)
        cfull[:m * ld].reshape(m, ld)[:, :n] = c0.reshape(m, n).float()
        cm = lambda t: gk.MatMut(t, m, n, ld, 1)  # noqa: E731
        got_of = lambda t: t[:m * ld].reshape(m, ld)[:, :n]  # noqa: E731
    c = cfull.to(dev)
    a = ai.to(torch.bfloat16).to(dev)
    b = bi.to(torch.bfloat16).to(dev)
    with tile(M16):
        gk.gemm_bf16_f32out(0.75, gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k), 0.5,
                            cm(c))
    got = c.cpu()
    assert torch.equal(got_of(got).double(), want), (m, k, n, layout)
    # the padding and the tail past C keep their fill
    if layout == "row424":
        assert (got[:m * ld].reshape(m, ld)[:, n:] == -7.0).all()
    tail = n * ld if layout == "col" else m * ld
    assert (got[tail:] == -7.0).all()
