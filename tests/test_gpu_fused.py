"""GPU parity of the fused bias/activation epilogue and the prepacked f32/bf16 RHS
(gemmkit's gemm_fused / gemm_batched_fused / gemm_packed_b_fused and
prepack_rhs / gemm_packed_b, src/api/fused.rs, src/api/batched.rs:307-590,
src/api/packed.rs:67-365, :684-950).

* f32: the fused result is bit-identical to the plain GEMM on the same inputs
  followed by the oracle's scalar map (the reference's own contract and test,
  tests/epilogue/float.rs:1-80), for every route: GEMV, skinny, matrix-core
  tiles, strided and padded C, both bias axes, every activation.
* bf16: the map runs in f32 before one narrowing, so the check is against the
  oracle (f64 product of the bf16 inputs, rounded to f32, then the bf16 map)
  within 1e-2 * max(|ref|, 1e-3 * max|ref|) elementwise.
* batched: each element is bit-identical to a standalone fused call;
  prepacked: bit-identical to the unpacked call (this engine's kernels read
  the packed copy in the same order).
* The reference's known answers: NaN -> +0, LeakyReLU(0) -> +0, and the
  degenerate k == 0 / alpha == 0 map C <- act(beta*C + bias).
"""
import numpy as np
import pytest
import torch

import gemmkit_amd as gk
import oracle
from helpers import bf16_tensor_from_bits, gather, layout_strides, scatter, to_dev

pytestmark = pytest.mark.gpu

ACTS = [(None, 0, 0.0), (gk.Activation.Relu, 1, 0.0), (gk.Activation.LeakyRelu(0.1), 2, 0.1)]


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def _operands(m, k, n, lc, seed):
    a = oracle.rand_vec(seed, m * k).astype(np.float32).reshape(m, k)
    b = oracle.rand_vec(seed + 1, k * n).astype(np.float32).reshape(k, n)
    c0 = oracle.rand_vec(seed + 2, m * n).astype(np.float32).reshape(m, n)
    rsc, csc, cl = layout_strides(m, n, lc, 3)
    return a, b, c0, (rsc, csc, cl)


def _run_f32(dev, alpha, a, b, beta, c0, cstr, bias=None, act=None, fused=True):
    m, k = a.shape
    n = b.shape[1]
    rsc, csc, cl = cstr
    cd = to_dev(scatter(c0, rsc, csc, cl, fill=np.float32(7.0)), dev)
    A = gk.MatRef.from_row_major(to_dev(a.ravel(), dev), m, k)
    B = gk.MatRef(to_dev(np.ascontiguousarray(b.T).ravel(), dev), k, n, 1, k)
    C = gk.MatMut(cd, m, n, rsc, csc)
    if fused:
        gk.gemm_fused(alpha, A, B, beta, C, bias, act)
    else:
        gk.gemm(alpha, A, B, beta, C)
    buf = cd.cpu().numpy()
    return gather(buf, m, n, rsc, csc), buf


# (m, k, n): the reference's driver shapes (tests/epilogue/float.rs:19-24) plus
# this engine's routes: GEMV (one short side), skinny (2..16), tile edges.
SHAPES = [(17, 17, 17), (33, 24, 40), (64, 64, 64), (48, 129, 96), (1, 300, 500),
          (700, 64, 1), (5, 256, 333), (300, 96, 12), (260, 200, 390)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_f32_fused_equals_gemm_then_map(dev, m, k, n):
    rng_b = oracle.rng_unit(m * 131 + n, m + n).astype(np.float32) * np.float32(3.0)
    brow, bcol = rng_b[:m].copy(), rng_b[m:].copy()
    case = 0
    for lc in ("col", "row", "col+"):
        for alpha, beta in ((1.0, 0.0), (0.9, 0.7), (1.0, 1.0)):
            a, b, c0, cstr = _operands(m, k, n, lc, 100 + case)
            case += 1
            plain, _ = _run_f32(dev, alpha, a, b, beta, c0, cstr, fused=False)
            for bias_kind in (0, 1, 2):
                for act, code, slope in ACTS:
                    if bias_kind == 0 and act is None:
                        continue
                    bt = None if bias_kind == 0 else to_dev(brow if bias_kind == 1 else bcol, dev)
                    bias = None if bt is None else (gk.Bias.PerRow(bt) if bias_kind == 1
                                                    else gk.Bias.PerCol(bt))
                    got, buf = _run_f32(dev, alpha, a, b, beta, c0, cstr, bias, act)
                    want = oracle.fused_map_f32(plain, None if bias_kind == 0 else
                                                (brow if bias_kind == 1 else bcol),
                                                bias_kind - 1 if bias_kind else 0, code, slope)
                    assert np.array_equal(_bits(got), _bits(want)), \
                        (lc, alpha, beta, bias_kind, code)
                    if lc == "col+":  # padding between columns untouched
                        rsc, csc, cl = cstr
                        mask = np.ones(cl, bool)
                        ii, jj = np.meshgrid(np.arange(m), np.arange(n), indexing="ij")
                        mask[(ii * rsc + jj * csc).ravel()] = False
                        assert (buf[mask] == np.float32(7.0)).all()


def test_f32_fused_unchecked_matches_checked(dev):
    # tests/epilogue/float.rs:478-560: the raw entry equals the checked one.
    m, k, n = 40, 72, 56
    a, b, c0, cstr = _operands(m, k, n, "col", 5)
    rsc, csc, cl = cstr
    bcol = to_dev(oracle.rng_unit(77, n).astype(np.float32), dev)
    act = gk.Activation.LeakyRelu(-0.3)
    checked, _ = _run_f32(dev, 0.9, a, b, 0.7, c0, cstr, gk.Bias.PerCol(bcol), act)
    cd = to_dev(scatter(c0, rsc, csc, cl), dev)
    ad = to_dev(a.ravel(), dev)
    bd = to_dev(np.ascontiguousarray(b.T).ravel(), dev)
    gk.gemm_fused_unchecked(m, k, n, 0.9, ad, k, 1, bd, 1, k, 0.7, cd, rsc, csc, bias=bcol,
                            bias_dim=gk.BIAS_PER_COL, act=act)
    raw = gather(cd.cpu().numpy(), m, n, rsc, csc)
    assert np.array_equal(_bits(raw), _bits(checked))
    # has_bias = false ignores the pointer.
    cd2 = to_dev(scatter(c0, rsc, csc, cl), dev)
    gk.gemm_fused_unchecked(m, k, n, 0.9, ad, k, 1, bd, 1, k, 0.7, cd2, rsc, csc, act=act)
    plain, _ = _run_f32(dev, 0.9, a, b, 0.7, c0, cstr, fused=False)
    want = oracle.fused_map_f32(plain, None, 0, 2, -0.3)
    assert np.array_equal(_bits(gather(cd2.cpu().numpy(), m, n, rsc, csc)), _bits(want))


@pytest.mark.parametrize("m,k,n", [(64, 2, 64), (1, 2, 64), (6, 2, 64)])
def test_nan_and_negative_zero(dev, m, k, n):
    # tests/epilogue/float.rs:274-358: inf + (-inf) = NaN maps to +0 under ReLU
    # and LeakyReLU; a zero product under a negative slope is +0.
    a = np.full((m, k), np.inf, np.float32)
    b = np.zeros((k, n), np.float32)
    b[0, :], b[1, :] = 1.0, -1.0
    for act in (gk.Activation.Relu, gk.Activation.LeakyRelu(0.25)):
        got, _ = _run_f32(dev, 1.0, a, b, 0.0, np.zeros((m, n), np.float32), (1, m, m * n),
                          act=act)
        assert (_bits(got) == 0).all()
    got, _ = _run_f32(dev, 1.0, np.zeros((m, k), np.float32), np.ones((k, n), np.float32), 0.0,
                      np.zeros((m, n), np.float32), (1, m, m * n),
                      act=gk.Activation.LeakyRelu(-0.5))
    assert (_bits(got) == 0).all()
    # bf16: same known answers through the narrowing store.
    ab = bf16_tensor_from_bits(oracle.bf16_bits(a).reshape(-1), dev)
    bb = bf16_tensor_from_bits(oracle.bf16_bits(np.ascontiguousarray(b.T)).reshape(-1), dev)
    cb = torch.zeros(m * n, dtype=torch.bfloat16, device=dev)
    gk.gemm_fused(1.0, gk.MatRef.from_row_major(ab, m, k), gk.MatRef(bb, k, n, 1, k), 0.0,
                  gk.MatMut(cb, m, n, 1, m), None, gk.Activation.Relu)
    assert (cb.view(torch.int16).cpu().numpy() == 0).all()


@pytest.mark.parametrize("k,alpha", [(0, 1.0), (24, 0.0)])
@pytest.mark.parametrize("lc", ["col", "row"])
def test_degenerate(dev, k, alpha, lc):
    # tests/epilogue/float.rs:361-395: C <- ReLU(beta*C0 + bias[i]), beta = 0.5,
    # element-wise in the user frame.
    m, n = 20, 24
    bias = oracle.rng_unit(0xDE6E, m).astype(np.float32)
    c0 = oracle.rng_unit(0xDE6F, m * n).astype(np.float32).reshape(m, n)
    rsc, csc, cl = layout_strides(m, n, lc)
    cd = to_dev(scatter(c0, rsc, csc, cl), dev)
    a = to_dev(np.ones(max(m * k, 1), np.float32), dev)
    b = to_dev(np.ones(max(k * n, 1), np.float32), dev)
    gk.gemm_fused(alpha, gk.MatRef(a, m, k, 1, m), gk.MatRef(b, k, n, 1, max(k, 1)), 0.5,
                  gk.MatMut(cd, m, n, rsc, csc), gk.Bias.PerRow(to_dev(bias, dev)),
                  gk.Activation.Relu)
    got = gather(cd.cpu().numpy(), m, n, rsc, csc)
    want = oracle.fused_map_f32(np.float32(0.5) * c0, bias, 0, 1)
    assert np.array_equal(_bits(got), _bits(want))
    # bf16: beta*C widened, the map in f32, one narrowing.
    cbits = oracle.bf16_bits(c0)
    bbits = oracle.bf16_bits(bias)
    cdb = bf16_tensor_from_bits(scatter(cbits.reshape(m, n), rsc, csc, cl), dev)
    ab = torch.zeros(max(m * k, 1), dtype=torch.bfloat16, device=dev)
    bb = torch.zeros(max(k * n, 1), dtype=torch.bfloat16, device=dev)
    gk.gemm_fused(alpha, gk.MatRef(ab, m, k, 1, m), gk.MatRef(bb, k, n, 1, max(k, 1)), 0.5,
                  gk.MatMut(cdb, m, n, rsc, csc), gk.Bias.PerRow(bf16_tensor_from_bits(bbits, dev)),
                  gk.Activation.LeakyRelu(0.25))
    got = gather(cdb.view(torch.int16).cpu().numpy().view(np.uint16), m, n, rsc, csc)
    base = np.float32(0.5) * oracle.bf16_to_f32(cbits).reshape(m, n)
    want = oracle.fused_map_bf16(base, bbits, 0, 2, 0x3E80)
    assert np.array_equal(got, want)


def _bf16_close(got_bits, want_bits):
    got = oracle.bf16_to_f32(got_bits).astype(np.float64)
    want = oracle.bf16_to_f32(want_bits).astype(np.float64)
    floor = 1e-3 * max(np.abs(want).max(), 1e-30)
    err = np.abs(got - want) / np.maximum(np.abs(want), floor)
    return float(err.max())


@pytest.mark.parametrize("m,k,n", [(17, 17, 17), (48, 129, 96), (1, 300, 500), (6, 128, 700),
                                   (260, 256, 390)])
@pytest.mark.parametrize("lc", ["col", "row"])
def test_bf16_fused_vs_oracle(dev, m, k, n, lc):
    a = oracle.bf16_bits(oracle.rng_normal(m + 3, m * k).astype(np.float32)).reshape(m, k)
    b = oracle.bf16_bits(oracle.rng_normal(n + 5, k * n).astype(np.float32)).reshape(k, n)
    c0 = oracle.bf16_bits(oracle.rng_normal(k + 7, m * n).astype(np.float32)).reshape(m, n)
    brow = oracle.bf16_bits(oracle.rng_unit(11, m).astype(np.float32) * 3)
    bcol = oracle.bf16_bits(oracle.rng_unit(12, n).astype(np.float32) * 3)
    alpha_b, beta_b = 0x3F66, 0x3F33  # bf16(0.9), bf16(0.7)
    alpha = float(oracle.bf16_to_f32(np.array([alpha_b]))[0])
    beta = float(oracle.bf16_to_f32(np.array([beta_b]))[0])
    rsc, csc, cl = layout_strides(m, n, lc)
    af, bf, cf = oracle.bf16_to_f32(a.ravel()), oracle.bf16_to_f32(b.ravel()), \
        oracle.bf16_to_f32(scatter(c0, rsc, csc, cl))
    ref = oracle.gemm_f64(m, k, n, alpha, af, k, 1, bf, n, 1, beta, cf, rsc, csc)
    ad = bf16_tensor_from_bits(a.ravel(), dev)
    bd = bf16_tensor_from_bits(np.ascontiguousarray(b.T).ravel(), dev)
    for bias_kind, bias_bits in ((1, brow), (2, bcol), (0, None)):
        for act, code, slope in ACTS[1:] + ([ACTS[0]] if bias_kind else []):
            cd = bf16_tensor_from_bits(scatter(c0, rsc, csc, cl), dev)
            bias = None
            if bias_kind:
                bt = bf16_tensor_from_bits(bias_bits, dev)
                bias = gk.Bias.PerRow(bt) if bias_kind == 1 else gk.Bias.PerCol(bt)
            gk.gemm_fused(alpha, gk.MatRef.from_row_major(ad, m, k), gk.MatRef(bd, k, n, 1, k),
                          beta, gk.MatMut(cd, m, n, rsc, csc), bias, act)
            got = gather(cd.view(torch.int16).cpu().numpy().view(np.uint16), m, n, rsc, csc)
            slope_bits = int(oracle.bf16_bits(np.array([slope], np.float32))[0])
            want = oracle.fused_map_bf16(ref.astype(np.float32), bias_bits,
                                         bias_kind - 1 if bias_kind else 0, code, slope_bits)
            assert _bf16_close(got, want) <= 1e-2, (bias_kind, code)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_batched_fused_equals_standalone(dev, dtype):
    # src/api/batched.rs:286-300: element e is bit-identical to a standalone
    # gemm_fused call; the bias is one shared vector.
    batch, m, k, n = 5, 40, 64, 72
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    g = torch.Generator(device="cpu").manual_seed(3)
    a = torch.randn(batch * m * k, generator=g).to(tdt).to(dev)
    b = torch.randn(batch * k * n, generator=g).to(tdt).to(dev)
    c0 = torch.randn(batch * m * n, generator=g).to(tdt).to(dev)
    bias = torch.randn(n, generator=g).to(tdt).to(dev)
    act = gk.Activation.LeakyRelu(0.2)
    c = c0.clone()
    gk.gemm_batched_fused(batch, 0.9, gk.MatRef.from_row_major(a, m, k), m * k,
                          gk.MatRef(b, k, n, 1, k), k * n, 0.5, gk.MatMut(c, m, n, 1, m), m * n,
                          gk.Bias.PerCol(bias), act)
    for e in range(batch):
        ce = c0[e * m * n:(e + 1) * m * n].clone()
        gk.gemm_fused(0.9, gk.MatRef.from_row_major(a[e * m * k:(e + 1) * m * k], m, k),
                      gk.MatRef(b[e * k * n:(e + 1) * k * n], k, n, 1, k), 0.5,
                      gk.MatMut(ce, m, n, 1, m), gk.Bias.PerCol(bias), act)
        assert torch.equal(ce.view(torch.int16 if dtype == "bf16" else torch.int32),
                           c[e * m * n:(e + 1) * m * n].view(torch.int16 if dtype == "bf16"
                                                             else torch.int32)), e
    # broadcast A (batch stride 0) through the raw entry
    c2 = c0.clone()
    gk.gemm_batched_fused_unchecked(batch, m, k, n, 0.9, a, k, 1, 0, b, 1, k, k * n, 0.5, c2, 1,
                                    m, m * n, bias=bias, bias_dim=gk.BIAS_PER_COL, act=act)
    ce = c0[m * n:2 * m * n].clone()
    gk.gemm_fused(0.9, gk.MatRef.from_row_major(a[:m * k], m, k),
                  gk.MatRef(b[k * n:2 * k * n], k, n, 1, k), 0.5, gk.MatMut(ce, m, n, 1, m),
                  gk.Bias.PerCol(bias), act)
    assert torch.equal(ce, c2[m * n:2 * m * n])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("m", [1, 8, 64, 300])
def test_packed_b_float(dev, dtype, m):
    # prepack_rhs / gemm_packed_b(_fused): column-major-ish C; results equal the
    # unpacked calls bit for bit.
    k, n = 200, 260
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    g = torch.Generator(device="cpu").manual_seed(m)
    a = torch.randn(m * k, generator=g).to(tdt).to(dev)
    b = torch.randn(k * n, generator=g).to(tdt).to(dev)
    c0 = torch.randn(m * n, generator=g).to(tdt).to(dev)
    bias = torch.randn(m, generator=g).to(tdt).to(dev)
    B = gk.MatRef.from_row_major(b, k, n)  # row-major B: the pack transposes it
    packed = gk.prepack_rhs(B)
    assert (packed.rows(), packed.cols()) == (k, n)
    A = gk.MatRef.from_row_major(a, m, k)
    ints = torch.int16 if dtype == "bf16" else torch.int32
    c1, c2 = c0.clone(), c0.clone()
    gk.gemm(0.5, A, B, 1.0, gk.MatMut(c1, m, n, 1, m))
    gk.gemm_packed_b(0.5, A, packed, 1.0, gk.MatMut(c2, m, n, 1, m))
    assert torch.equal(c1.view(ints), c2.view(ints))
    c3, c4 = c0.clone(), c0.clone()
    act = gk.Activation.Relu
    gk.gemm_fused(0.5, A, B, 1.0, gk.MatMut(c3, m, n, 1, m), gk.Bias.PerRow(bias), act)
    gk.gemm_packed_b_fused(0.5, A, packed, 1.0, gk.MatMut(c4, m, n, 1, m), gk.Bias.PerRow(bias),
                           act)
    assert torch.equal(c3.view(ints), c4.view(ints))
    c5 = c0.clone()
    gk.gemm_packed_b_fused_unchecked(0.5, m, a, k, 1, packed, 1.0, c5, 1, m, bias=bias,
                                     bias_dim=gk.BIAS_PER_ROW, act=act)
    assert torch.equal(c3.view(ints), c5.view(ints))
    # row-major C is refused, as in the reference (src/api/packed.rs:625-629)
    if m > 1:
        with pytest.raises(gk.GemmkitError) as e:
            gk.gemm_packed_b(0.5, A, packed, 1.0, gk.MatMut.from_row_major(c0.clone(), m, n))
        assert "column-major-ish C" in str(e.value)


def test_packed_handle_type_is_checked(dev):
    b = torch.zeros(64 * 32, device=dev)
    packed = gk.prepack_rhs(gk.MatRef.from_row_major(b, 64, 32))
    a = torch.zeros(8 * 64, dtype=torch.int8, device=dev)
    c = torch.zeros(8 * 32, dtype=torch.int32, device=dev)
    with pytest.raises(gk.GemmkitError) as e:
        gk.gemm_i8_packed_b(1, gk.MatRef.from_row_major(a, 8, 64), packed, 0,
                            gk.MatMut(c, 8, 32, 1, 8))
    assert str(e.value) == "gemmkit: packed RHS holds f32 elements, this entry takes i8"
