"""GPU parity: f32 and bf16 GEMM, batched GEMM and GEMV against the oracle's
f64 closed form, within the stated tolerances:

* f32: relative Frobenius error ||got - ref||_F / ||ref||_F <= 1e-5 (and the
  reference's own gate ||got - ref||_F / (||A||_F ||B||_F) <= 8 k eps,
  tests/oracle_common/mod.rs:185-217);
* bf16 with f32 output: elementwise |got - ref| <= 1e-2 * max(|ref|, 1e-3 * max|ref|)
  against the f64 product of the bf16-rounded inputs;
* bf16 output (the reference's gemm::<bf16>, src/kernel/mixed.rs:96-200): within
  one bf16 rounding of the f64 reference (relative 2^-8, same floor);
* batched: every element equal, bitwise, to a standalone call on that element
  (tests/batched.rs:1-3).
"""
import numpy as np
import pytest

import gemmkit_amd as gk
import oracle
from helpers import rel_errors, bf16_tensor_from_bits, gather, layout_strides, scatter, to_dev

pytestmark = pytest.mark.gpu

F32_EPS = np.finfo(np.float32).eps


def rel_frob(got, ref):
    return float(np.linalg.norm((got - ref).ravel()) / max(np.linalg.norm(ref.ravel()), 1e-300))


def test_readme_2x2(dev):
    # README.md:55-71 / src/lib.rs:9-25: [1..6] . [7..12] = [58, 64, 139, 154]
    import torch
    a = to_dev(np.arange(1, 7, dtype=np.float32), dev)
    b = to_dev(np.arange(7, 13, dtype=np.float32), dev)
    c = torch.zeros(4, device=dev)
    gk.gemm(1.0, gk.MatRef.from_row_major(a, 2, 3), gk.MatRef.from_row_major(b, 3, 2), 0.0,
            gk.MatMut.from_row_major(c, 2, 2))
    assert c.cpu().tolist() == [58.0, 64.0, 139.0, 154.0]


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (2, 3, 2), (17, 33, 9), (64, 64, 64),
                                   (100, 257, 130), (512, 512, 512), (300, 1000, 700),
                                   (1, 5000, 300), (300, 5000, 1), (1000, 64, 3)])
@pytest.mark.parametrize("la,lb,lc", [("row", "row", "row"), ("row", "col", "row"),
                                      ("col", "col", "col"), ("row+", "col+", "col+")])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.75, -1.5)])
def test_f32(dev, m, k, n, la, lb, lc, alpha, beta):
    a = oracle.rand_vec(1 + m, m * k).astype(np.float32).reshape(m, k)
    b = oracle.rand_vec(2 + n, k * n).astype(np.float32).reshape(k, n)
    c0 = oracle.rand_vec(3 + k, m * n).astype(np.float32).reshape(m, n)
    rsa, csa, al = layout_strides(m, k, la, 3)
    rsb, csb, bl = layout_strides(k, n, lb, 3)
    rsc, csc, cl = layout_strides(m, n, lc, 3)
    abuf, bbuf, cbuf = scatter(a, rsa, csa, al), scatter(b, rsb, csb, bl), scatter(c0, rsc, csc, cl)
    ref = oracle.gemm_f64(m, k, n, alpha, abuf, rsa, csa, bbuf, rsb, csb, beta, cbuf, rsc, csc)
    cd = to_dev(cbuf, dev)
    gk.gemm(alpha, gk.MatRef(to_dev(abuf, dev), m, k, rsa, csa),
            gk.MatRef(to_dev(bbuf, dev), k, n, rsb, csb), beta, gk.MatMut(cd, m, n, rsc, csc))
    got = gather(cd.cpu().numpy(), m, n, rsc, csc).astype(np.float64)
    assert rel_frob(got, ref) <= 1e-5
    # the reference's own gate
    num = np.linalg.norm((got - ref).ravel())
    den = np.linalg.norm(a.ravel()) * np.linalg.norm(b.ravel()) * abs(alpha) + \
        abs(beta) * np.linalg.norm(c0.ravel()) + 1e-30
    assert num / den <= 8 * max(k, 1) * F32_EPS


def test_f32_gemv_16384(dev):
    """The f32 GEMV workload at full size (16384 x 16384 row-major times a vector)."""
    import torch
    n = 16384
    g = torch.Generator(device="cpu").manual_seed(5)
    A = torch.randn(n * n, generator=g)
    x = torch.randn(n, generator=g)
    ref = oracle.gemv_f64(n, n, 1.0, A.numpy(), n, 1, x.numpy(), 1)
    y = torch.empty(n, device=dev)
    gk.gemm(1.0, gk.MatRef.from_row_major(A.to(dev), n, n), gk.MatRef(x.to(dev), n, 1, 1, 1),
            0.0, gk.MatMut(y, n, 1, 1, 1))
    assert rel_frob(y.cpu().numpy().astype(np.float64), ref) <= 1e-5


def _bf16(x):
    bits = oracle.bf16_bits(x.astype(np.float32))
    return bits, oracle.bf16_to_f32(bits)


@pytest.mark.parametrize("m,k,n", [(1, 16, 1), (5, 40, 7), (64, 128, 64), (130, 200, 250),
                                   (512, 128, 512), (777, 1024, 333), (4, 4096, 1000)])
@pytest.mark.parametrize("la,lb", [("row", "col"), ("row", "row"), ("col+", "row+")])
def test_bf16_f32out(dev, m, k, n, la, lb, record_property):
    import torch
    abits, af = _bf16(oracle.rng_normal(11 + m, m * k))
    bbits, bf = _bf16(oracle.rng_normal(12 + n, k * n))
    rsa, csa, al = layout_strides(m, k, la, 8)
    rsb, csb, bl = layout_strides(k, n, lb, 8)
    abuf = scatter(abits.reshape(m, k), rsa, csa, al)
    bbuf = scatter(bbits.reshape(k, n), rsb, csb, bl)
    alpha = 1.0 / np.sqrt(128.0)
    ref = oracle.gemm_f64(m, k, n, alpha, af, k, 1, bf, n, 1)
    c = torch.empty(m * n, dtype=torch.float32, device=dev)
    gk.gemm_bf16_f32out(alpha, gk.MatRef(bf16_tensor_from_bits(abuf, dev), m, k, rsa, csa),
                        gk.MatRef(bf16_tensor_from_bits(bbuf, dev), k, n, rsb, csb), 0.0,
                        gk.MatMut.from_row_major(c, m, n))
    got = c.cpu().numpy().reshape(m, n).astype(np.float64)
    floored, unfloored = rel_errors(got, ref)
    # the gate is floored at 1e-3 max|ref| (f32 accumulation cannot bound the
    # relative error of an output that cancels to near zero); the unfloored
    # maximum is reported beside it
    record_property("bf16_rel_err_floored_max", floored)
    record_property("bf16_rel_err_unfloored_max", unfloored)
    print(f"bf16->f32 {m}x{k}x{n} {la}/{lb}: max rel err floored {floored:.3g}, "
          f"unfloored {unfloored:.3g}")
    assert floored <= 1e-2


@pytest.mark.parametrize("m,k,n", [(3, 8, 5), (64, 128, 64), (300, 300, 300)])
def test_bf16_out(dev, m, k, n):
    """gemm::<bf16>: f32 accumulate, alpha*acc + beta*C, one RNE narrowing."""
    import torch
    abits, af = _bf16(oracle.rng_normal(21 + m, m * k))
    bbits, bf = _bf16(oracle.rng_normal(22 + n, k * n))
    cbits, cf = _bf16(oracle.rng_normal(23 + k, m * n))
    alpha, beta = 0.5, 2.0  # exact in bf16
    ref = oracle.gemm_f64(m, k, n, alpha, af, k, 1, bf, n, 1, beta, cf, n, 1)
    cd = bf16_tensor_from_bits(cbits, dev)
    gk.gemm(alpha, gk.MatRef.from_row_major(bf16_tensor_from_bits(abits, dev), m, k),
            gk.MatRef.from_row_major(bf16_tensor_from_bits(bbits, dev), k, n), beta,
            gk.MatMut.from_row_major(cd, m, n))
    got = cd.float().cpu().numpy().reshape(m, n).astype(np.float64)
    floor = 1e-3 * np.abs(ref).max()
    assert (np.abs(got - ref) <= 2.0 ** -8 * np.maximum(np.abs(ref), floor) * 1.01).all()


@pytest.mark.parametrize("m,n", [(512, 512), (512, 8), (1, 512)])
@pytest.mark.parametrize("alpha", [1.0, 0.3])
def test_bf16_out_rounding_bit_exact(dev, m, n, alpha):
    """One nonzero product per output (k = 8, a single nonzero column of A and
    row of B), so the f32 value before narrowing is known exactly:
    f32(alpha * a_i * b_j), alpha being a bf16 scalar like the operands
    (gemm::<bf16> takes alpha: bf16).  Its bf16 bits must equal the oracle's
    RNE with gemmkit's NaN rule, ties included (products of two bf16 carry up
    to 16 significant bits)."""
    k = 8
    rng = np.random.default_rng(7 + m + n)

    def bf16_vals(cnt):
        mant = rng.integers(0, 128, cnt)
        expo = rng.integers(-20, 21, cnt)
        sign = rng.choice([-1.0, 1.0], cnt)
        return (sign * (1.0 + mant / 128.0) * np.exp2(expo)).astype(np.float32)

    av, bv = bf16_vals(m), bf16_vals(n)
    a = np.zeros((m, k), np.float32)
    b = np.zeros((k, n), np.float32)
    a[:, 3], b[3, :] = av, bv
    alpha_bf = oracle.bf16_to_f32(oracle.bf16_bits(np.array([alpha], np.float32)))[0]
    want = oracle.bf16_bits(alpha_bf * (av[:, None] * bv[None, :]).astype(np.float32))
    cd = bf16_tensor_from_bits(np.zeros(m * n, np.uint16), dev)
    gk.gemm(alpha, gk.MatRef.from_row_major(bf16_tensor_from_bits(oracle.bf16_bits(a), dev), m, k),
            gk.MatRef.from_row_major(bf16_tensor_from_bits(oracle.bf16_bits(b), dev), k, n), 0.0,
            gk.MatMut.from_row_major(cd, m, n))
    import torch
    got = cd.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, want.reshape(-1))


def _narrow_case(dev, av, bv, alpha):
    """bf16 GEMM with one nonzero product per output: returns (got bits, want
    bits), want = RNE(f32(alpha) * f32(a_i * b_j)) with gemmkit's NaN rule, the
    f32 values computed by numpy (IEEE, subnormals kept)."""
    import torch
    m, n, k = av.size, bv.size, 8
    a = np.zeros((m, k), np.float32)
    b = np.zeros((k, n), np.float32)
    a[:, 5], b[5, :] = av, bv
    assert np.array_equal(oracle.bf16_to_f32(oracle.bf16_bits(a)), a.ravel())
    assert np.array_equal(oracle.bf16_to_f32(oracle.bf16_bits(b)), b.ravel())
    alpha_bf = np.float32(oracle.bf16_to_f32(oracle.bf16_bits(np.array([alpha], np.float32)))[0])
    assert alpha_bf == np.float32(alpha)
    with np.errstate(over="ignore"):
        v = alpha_bf * (av[:, None] * bv[None, :]).astype(np.float32)
    want = oracle.bf16_bits(v)
    cd = bf16_tensor_from_bits(np.zeros(m * n, np.uint16), dev)
    gk.gemm(alpha, gk.MatRef.from_row_major(bf16_tensor_from_bits(oracle.bf16_bits(a), dev), m, k),
            gk.MatRef.from_row_major(bf16_tensor_from_bits(oracle.bf16_bits(b), dev), k, n), 0.0,
            gk.MatMut.from_row_major(cd, m, n))
    got = cd.view(torch.int16).cpu().numpy().view(np.uint16)
    return got, want.reshape(-1), v.ravel()


def _mantissas(rng, cnt):
    """bf16 significands 1.xxxxxxx as integers 128..255 over 128."""
    return rng.integers(128, 256, cnt).astype(np.float64) / 128.0


@pytest.mark.parametrize("m,n", [(512, 512), (512, 8), (1, 512)])
def test_bf16_out_narrowing_subnormal_results(dev, m, n):
    """f32 results below 2^-126 (subnormal) narrowed to bf16: alpha = 2^-40
    scales exact products of about 2^-100 into [2^-147, 2^-127].  The scaling
    multiply itself rounds onto the f32 subnormal grid (IEEE round to nearest
    even: numpy on the host, the kernel's f32 multiply on the device, which
    must keep subnormals), then the narrowing rounds again; the grid holds
    constructed ties (f32 bits 0x8000 and 0x18000) and results that round to
    the smallest bf16 subnormal or to zero."""
    rng = np.random.default_rng(100 + m + n)
    sa = rng.choice([-1.0, 1.0], m)
    sb = rng.choice([-1.0, 1.0], n)
    av = (sa * _mantissas(rng, m) * np.exp2(rng.integers(-55, -48, m))).astype(np.float32)
    bv = (sb * _mantissas(rng, n) * np.exp2(rng.integers(-52, -45, n))).astype(np.float32)
    if m >= 2 and n >= 2:
        # 2^-134 and 3 * 2^-134 are f32 bits 0x8000 and 0x18000: ties that
        # round to the even 0x0000 and 0x0002; 5 * 2^-136 (0xA000) rounds up
        av[:2] = [1.0 * 2.0 ** -50, 3.0 * 2.0 ** -50]
        bv[:2] = [1.0 * 2.0 ** -44, 5.0 * 2.0 ** -46]
    got, want, v = _narrow_case(dev, av, bv, 2.0 ** -40)
    sub = np.abs(v) < np.float32(2.0 ** -126)
    assert sub.mean() > 0.5  # most results really are subnormal
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (f"{bad.size} mismatches, first {bad[:4]}: got {got[bad[:4]]} "
                           f"want {want[bad[:4]]} from f32 {v[bad[:4]]}")


@pytest.mark.parametrize("m,n", [(512, 512), (512, 8), (1, 512)])
def test_bf16_out_narrowing_top_exponent_and_overflow(dev, m, n):
    """f32 results in [2^126, 2^128) and beyond narrowed to bf16: values at or
    above the midpoint between the largest bf16 (0x7F7F) and infinity round to
    +-inf, the midpoint itself (0x7F7F8000, a tie to the even 0x7F80) included;
    the tie 0x7F7E8000 rounds to 0x7F7E; products past the f32 range are +-inf
    already.  alpha = 2^19 scales exact products of about 2^108."""
    rng = np.random.default_rng(200 + m + n)
    sa = rng.choice([-1.0, 1.0], m)
    sb = rng.choice([-1.0, 1.0], n)
    av = (sa * _mantissas(rng, m) * np.exp2(rng.integers(53, 56, m))).astype(np.float32)
    bv = (sb * _mantissas(rng, n) * np.exp2(rng.integers(52, 55, n))).astype(np.float32)
    # 73 * 7 = 511 = 0x1FF: 511 * 2^119 is f32 0x7F7F8000, the midpoint to
    # infinity (and its negative); 127 * 4 * 2^119 is the largest bf16 exactly
    av[0] = 73.0 * 2.0 ** 60
    bv[:3] = [7.0 * 2.0 ** 40, -7.0 * 2.0 ** 40, 4.0 * 2.0 ** 40][:n]
    if m >= 3:
        av[1:3] = [-73.0 * 2.0 ** 60, 127.0 * 2.0 ** 60]
    got, want, v = _narrow_case(dev, av, bv, 2.0 ** 19)
    top = np.abs(v) >= np.float32(2.0 ** 126)
    assert top.mean() > 0.3
    assert (np.isinf(oracle.bf16_to_f32(want))).any()  # some really round to infinity
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (f"{bad.size} mismatches, first {bad[:4]}: got {got[bad[:4]]} "
                           f"want {want[bad[:4]]} from f32 {v[bad[:4]]}")


def test_batched_bf16_attention_scores(dev):
    """Batched bf16 x bf16 -> f32, the attention-score shape at full size:
    64 x (512 x 128) . (128 x 512) with B = K^T via strides, alpha = 1/sqrt(128).
    Each element is checked against the f64 closed form (sampled elements) and
    equal bitwise to a standalone gemm_bf16_f32out on that element."""
    import torch
    Bt, S, D = 64, 512, 128
    qbits, qf = _bf16(oracle.rng_normal(31, Bt * S * D))
    kbits, kf = _bf16(oracle.rng_normal(32, Bt * S * D))
    q, kk = bf16_tensor_from_bits(qbits, dev), bf16_tensor_from_bits(kbits, dev)
    out = torch.empty(Bt * S * S, dtype=torch.float32, device=dev)
    alpha = 1.0 / np.sqrt(128.0)
    gk.gemm_batched_bf16_f32out(Bt, alpha, gk.MatRef.from_row_major(q, S, D), S * D,
                                gk.MatRef(kk, D, S, 1, D), S * D, 0.0,
                                gk.MatMut.from_row_major(out, S, S), S * S)
    got = out.cpu().numpy()
    for z in (0, 17, 63):
        ref = oracle.gemm_f64(S, D, S, alpha, qf[z * S * D:], D, 1, kf[z * S * D:], 1, D)
        g = got[z * S * S:(z + 1) * S * S].reshape(S, S).astype(np.float64)
        floor = 1e-3 * np.abs(ref).max()
        assert (np.abs(g - ref) <= 1e-2 * np.maximum(np.abs(ref), floor)).all(), z
        one = torch.empty(S * S, dtype=torch.float32, device=dev)
        gk.gemm_bf16_f32out(alpha, gk.MatRef.from_row_major(q[z * S * D:(z + 1) * S * D], S, D),
                            gk.MatRef(kk[z * S * D:(z + 1) * S * D], D, S, 1, D), 0.0,
                            gk.MatMut.from_row_major(one, S, S))
        assert np.array_equal(one.cpu().numpy().view(np.uint32),
                              got[z * S * S:(z + 1) * S * S].view(np.uint32)), z


@pytest.mark.parametrize("batch,m,k,n,a_bs0,b_bs0", [(5, 33, 40, 21, False, False),
                                                     (8, 64, 64, 64, True, False),
                                                     (3, 100, 257, 60, False, True)])
def test_batched_f32_equals_loop(dev, batch, m, k, n, a_bs0, b_bs0):
    # tests/batched.rs:30-80: batched == loop of gemm, bitwise; a stride of 0 broadcasts
    import torch
    a_bs = 0 if a_bs0 else m * k
    b_bs = 0 if b_bs0 else k * n
    a = torch.from_numpy(oracle.rand_vec(41, max(a_bs * batch, m * k)).astype(np.float32)).to(dev)
    b = torch.from_numpy(oracle.rand_vec(42, max(b_bs * batch, k * n)).astype(np.float32)).to(dev)
    c = torch.zeros(batch * m * n, device=dev)
    gk.gemm_batched(batch, 1.25, gk.MatRef.from_row_major(a, m, k), a_bs,
                    gk.MatRef.from_row_major(b, k, n), b_bs, 0.0,
                    gk.MatMut.from_row_major(c, m, n), m * n)
    for z in range(batch):
        one = torch.zeros(m * n, device=dev)
        gk.gemm(1.25, gk.MatRef.from_row_major(a[z * a_bs:z * a_bs + m * k], m, k),
                gk.MatRef.from_row_major(b[z * b_bs:z * b_bs + k * n], k, n), 0.0,
                gk.MatMut.from_row_major(one, m, n))
        assert torch.equal(one, c[z * m * n:(z + 1) * m * n]), z
        ref = oracle.gemm_f64(m, k, n, 1.25, a[z * a_bs:].cpu().numpy(), k, 1,
                              b[z * b_bs:].cpu().numpy(), n, 1)
        assert rel_frob(one.cpu().numpy().reshape(m, n).astype(np.float64), ref) <= 1e-5


def test_batched_bf16_out_equals_loop(dev):
    import torch
    batch, m, k, n = 4, 70, 96, 50
    abits, _ = _bf16(oracle.rng_normal(51, batch * m * k))
    bbits, _ = _bf16(oracle.rng_normal(52, batch * k * n))
    a, b = bf16_tensor_from_bits(abits, dev), bf16_tensor_from_bits(bbits, dev)
    c = torch.zeros(batch * m * n, dtype=torch.bfloat16, device=dev)
    gk.gemm_batched(batch, 1.0, gk.MatRef.from_row_major(a, m, k), m * k,
                    gk.MatRef.from_row_major(b, k, n), k * n, 0.0,
                    gk.MatMut.from_row_major(c, m, n), m * n)
    for z in range(batch):
        one = torch.zeros(m * n, dtype=torch.bfloat16, device=dev)
        gk.gemm(1.0, gk.MatRef.from_row_major(a[z * m * k:(z + 1) * m * k], m, k),
                gk.MatRef.from_row_major(b[z * k * n:(z + 1) * k * n], k, n), 0.0,
                gk.MatMut.from_row_major(one, m, n))
        assert torch.equal(one.view(torch.int16), c[z * m * n:(z + 1) * m * n].view(torch.int16))
