"""GPU parity for the skinny route (products with a short side of 1..16).

Short sides of 2..16 run on the matrix-core skinny kernel (vectors staged in
LDS); a short side of 1, or up to 8 with GEMMKIT_HIP_SKINNY=0, runs on the
wavefront-reduction GEMV.  i8 and requantized outputs are bit-exact against
the oracle and identical between the two kernels; f32 and bf16 meet the
tolerances of the float suite.  Includes the decode-shaped workload at full
size: W 14336 x 4096 i8 times M = 1 and 8 activation rows.
"""
import os

import numpy as np
import pytest

import gemmkit_amd as gk
import oracle
from helpers import gather, layout_strides, scatter, to_dev
from test_gpu_float import rel_frob
from test_gpu_i8 import run_case
from test_gpu_requant import _run as run_requant

pytestmark = pytest.mark.gpu


class no_skinny:
    """Context: route short sides 2..8 to the wavefront GEMV instead."""

    def __enter__(self):
        os.environ["GEMMKIT_HIP_SKINNY"] = "0"

    def __exit__(self, *exc):
        os.environ.pop("GEMMKIT_HIP_SKINNY", None)


I8_CASES = [
    # (m, k, n): short side on m, then on n; K multiples of 16, ragged K, long K
    (1, 16, 1), (1, 64, 100), (2, 48, 33), (3, 1040, 31), (5, 4096, 1000), (8, 100, 257),
    (9, 4096, 64), (12, 640, 129), (16, 4112, 300), (16, 16, 16),
    (100, 64, 1), (257, 48, 2), (1000, 4096, 7), (33, 1040, 12), (300, 4112, 16),
    # one vector, 1..8 KiB rows (4, 4, 2 and 1 rows per wave iteration), ragged row counts
    (1, 1024, 257), (1, 2048, 1001), (1, 4096, 3), (1, 8192, 301), (1001, 8192, 1),
    # one vector, rows past 8 KiB (the streaming kernel): whole batches only, and a
    # ragged last batch
    (1, 16384, 513), (1, 20000, 300), (700, 20000, 1),
]


@pytest.mark.parametrize("m,k,n", I8_CASES)
@pytest.mark.parametrize("alpha,beta", [(1, 0), (3, -2)])
def test_i8_skinny(dev, m, k, n, alpha, beta):
    run_case(dev, m, k, n, alpha, beta, "row", "col", "row", seed=11)


@pytest.mark.parametrize("m,k,n", [(4, 200, 300), (300, 96, 6), (16, 1000, 70)])
@pytest.mark.parametrize("la,lb,lc", [("col", "col", "col"), ("row", "row", "row"),
                                      ("row+", "col+", "col+")])
def test_i8_skinny_layouts(dev, m, k, n, la, lb, lc):
    run_case(dev, m, k, n, 2, 1, la, lb, lc, seed=12)


@pytest.mark.parametrize("m,k,n", [(2, 1040, 777), (8, 4096, 1000), (6, 4112, 300),
                                   (500, 1040, 3), (2, 4096, 777)])
def test_i8_skinny_matches_gemv(dev, m, k, n):
    """Both skinny kernels give identical bits (wrapping i32 sums); (2, 4096)
    takes the wavefront GEMV on both runs (two vectors with 4 KiB rows)."""
    run_case(dev, m, k, n, 1, 0, "row", "col", "row", seed=13)
    with no_skinny():
        run_case(dev, m, k, n, 1, 0, "row", "col", "row", seed=13)


@pytest.mark.parametrize("m", [1, 8])
def test_decode_gemv_full_size(dev, m):
    """W 14336 x 4096 (B = W^T, column-major view) times M activation rows."""
    import torch
    nw, k = 14336, 4096
    w = oracle.rng_i8_sym127(31, nw * k)
    x = oracle.rng_i8_sym127(32 + m, m * k)
    want = np.zeros(m * nw, np.int32)
    oracle.gemm_i8(m, k, nw, 1, x, k, 1, w, 1, k, 0, want, nw, 1)
    c = torch.empty(m * nw, dtype=torch.int32, device=dev)
    gk.gemm_i8(1, gk.MatRef.from_row_major(to_dev(x, dev), m, k),
               gk.MatRef(to_dev(w, dev), k, nw, 1, k), 0, gk.MatMut.from_row_major(c, m, nw))
    assert np.array_equal(c.cpu().numpy(), want)


@pytest.mark.parametrize("m,k,n", [(1, 5000, 300), (300, 5000, 1), (4, 1000, 513), (700, 64, 16),
                                   (16, 2048, 200), (7, 3, 90),
                                   # 2..4 vectors with 4..8 KiB rows: the wavefront GEMV
                                   (2, 1024, 700), (3, 2048, 301), (600, 1536, 4), (4, 2048, 64),
                                   # one vector, 4 and 8 KiB rows, ragged row counts
                                   (1, 1024, 3), (1, 2048, 257), (513, 2048, 1),
                                   # rows past 8 KiB, ragged last batch
                                   (1, 16400, 129), (2, 9000, 77)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.75, -1.5)])
def test_f32_skinny(dev, m, k, n, alpha, beta):
    a = oracle.rand_vec(41 + m, m * k).astype(np.float32).reshape(m, k)
    b = oracle.rand_vec(42 + n, k * n).astype(np.float32).reshape(k, n)
    c0 = oracle.rand_vec(43 + k, m * n).astype(np.float32).reshape(m, n)
    rsa, csa, al = layout_strides(m, k, "row", 0)
    rsb, csb, bl = layout_strides(k, n, "col", 0)
    rsc, csc, cl = layout_strides(m, n, "row", 0)
    abuf, bbuf, cbuf = scatter(a, rsa, csa, al), scatter(b, rsb, csb, bl), scatter(c0, rsc, csc, cl)
    ref = oracle.gemm_f64(m, k, n, alpha, abuf, rsa, csa, bbuf, rsb, csb, beta, cbuf, rsc, csc)
    cd = to_dev(cbuf, dev)
    gk.gemm(alpha, gk.MatRef(to_dev(abuf, dev), m, k, rsa, csa),
            gk.MatRef(to_dev(bbuf, dev), k, n, rsb, csb), beta, gk.MatMut(cd, m, n, rsc, csc))
    got = gather(cd.cpu().numpy(), m, n, rsc, csc).astype(np.float64)
    assert rel_frob(got, ref) <= 1e-5


@pytest.mark.parametrize("m,k,n", [(1, 4096, 1000), (8, 2048, 333), (300, 512, 12),
                                   (1, 12000, 300)])
def test_bf16_f32out_skinny(dev, m, k, n):
    import torch
    g = torch.Generator().manual_seed(m * 1000 + n)
    a = torch.randn(m * k, generator=g).to(torch.bfloat16)
    b = torch.randn(n * k, generator=g).to(torch.bfloat16)  # B given transposed: n x k
    c = torch.empty(m * n, dtype=torch.float32, device=dev)
    gk.gemm_bf16_f32out(1.0, gk.MatRef.from_row_major(a.to(dev), m, k),
                        gk.MatRef(b.to(dev), k, n, 1, k), 0.0, gk.MatMut.from_row_major(c, m, n))
    ref = a.double().reshape(m, k) @ b.double().reshape(n, k).T
    got = c.cpu().double().reshape(m, n)
    floor = 1e-3 * ref.abs().max().item()
    assert torch.all((got - ref).abs() <= 1e-2 * torch.clamp(ref.abs(), min=floor))


@pytest.mark.parametrize("m,k,n,axis", [(6, 4096, 1000, 1), (6, 4096, 1000, 0),
                                        (1000, 512, 5, 0), (1000, 512, 5, 1), (16, 1040, 77, 1)])
@pytest.mark.parametrize("relu", [False, True])
def test_requant_skinny(dev, m, k, n, axis, relu):
    """Per-channel scale and bias on both axes: the route swaps operands when
    the short side is N, which flips the channel axis."""
    a = oracle.rng_i8_sym127(500 + m, m * k)
    b = oracle.rng_i8_sym127(600 + n, k * n)
    ch = n if axis else m
    u = oracle.rng_unit(700 + ch, 2 * ch)
    scales = (1e-4 + (u[:ch] + 1) / 2 * (1e-2 - 1e-4)).astype(np.float32)
    bias = np.round(u[ch:] * 65536).astype(np.int32)
    got, want = run_requant(dev, m, k, n, a, b, k, 1, 1, k, 0.0, scales, 0, bias, axis, relu,
                            False, n, 1, m * n)
    assert np.array_equal(got, want)


# Many rows (8192 and up, the decode weights' size): ragged rows, ragged and
# long K, 3..16 vectors, vectors row-major and strided, alpha/beta.
WHOLE_ROWS = [(3, 1000, 8200), (8, 4096, 10001), (16, 260, 8193), (5, 4112, 9000),
              (8, 4096, 14336), (12, 96, 8192)]


@pytest.mark.parametrize("m,k,n", WHOLE_ROWS)
@pytest.mark.parametrize("la", ["row", "col"])
@pytest.mark.parametrize("alpha,beta", [(1, 0), (3, -2)])
def test_i8_whole_rows(dev, m, k, n, la, alpha, beta):
    run_case(dev, m, k, n, alpha, beta, la, "col", "row", seed=13)


@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("relu", [False, True])
def test_requant_whole_rows(dev, axis, relu):
    m, k, n = 7, 2064, 9001
    a = oracle.rng_i8_sym127(510 + m, m * k)
    b = oracle.rng_i8_sym127(610 + n, k * n)
    ch = n if axis else m
    u = oracle.rng_unit(710 + ch, 2 * ch)
    scales = (1e-4 + (u[:ch] + 1) / 2 * (1e-2 - 1e-4)).astype(np.float32)
    bias = np.round(u[ch:] * 65536).astype(np.int32)
    got, want = run_requant(dev, m, k, n, a, b, k, 1, 1, k, 0.0, scales, 3, bias, axis, relu,
                            False, n, 1, m * n)
    assert np.array_equal(got, want)


def test_batched_skinny_equals_loop(dev):
    """Batched products with a short side of 4: each element bit-equal to a
    standalone call."""
    import torch
    batch, m, k, n = 6, 4, 640, 300
    g = torch.Generator().manual_seed(9)
    a = torch.randn(batch * m * k, generator=g).to(torch.bfloat16).to(dev)
    b = torch.randn(batch * n * k, generator=g).to(torch.bfloat16).to(dev)
    c = torch.empty(batch * m * n, dtype=torch.float32, device=dev)
    gk.gemm_batched_bf16_f32out(batch, 0.5, gk.MatRef.from_row_major(a, m, k), m * k,
                                gk.MatRef(b, k, n, 1, k), n * k, 0.0,
                                gk.MatMut.from_row_major(c, m, n), m * n)
    for z in range(batch):
        one = torch.empty(m * n, dtype=torch.float32, device=dev)
        gk.gemm_bf16_f32out(0.5, gk.MatRef.from_row_major(a[z * m * k:], m, k),
                            gk.MatRef(b[z * n * k:], k, n, 1, k), 0.0,
                            gk.MatMut.from_row_major(one, m, n))
        assert torch.equal(one, c[z * m * n:(z + 1) * m * n])


@pytest.mark.parametrize("dtype", ["i8", "f32", "bf16"])
@pytest.mark.parametrize("m", [2, 8, 16])
def test_strided_vectors_small_batch(dev, dtype, m):
    """gemmkit's fixed-weight inference shape (benches/gemm_bench.rs:380-470):
    A (m x 2048) column-major -- vectors staged element by element, no pack --
    against a 2048 x 2048 weight, plain and prepacked, C column-major."""
    import torch
    k = n = 2048
    tdt = {"i8": torch.int8, "f32": torch.float32, "bf16": torch.bfloat16}[dtype]
    g = torch.Generator().manual_seed(m)
    if dtype == "i8":
        a = torch.randint(-128, 128, (m * k,), dtype=torch.int8, generator=g)
        b = torch.randint(-128, 128, (k * n,), dtype=torch.int8, generator=g)
    else:
        a = torch.randn(m * k, generator=g).to(tdt)
        b = torch.randn(k * n, generator=g).to(tdt)
    ad, bd = a.to(dev), b.to(dev)
    A = gk.MatRef.from_col_major(ad, m, k)
    if dtype == "i8":
        B = gk.MatRef.from_col_major(bd, k, n)
        c1 = torch.zeros(m * n, dtype=torch.int32, device=dev)
        c2 = torch.zeros_like(c1)
        gk.gemm_i8(1, A, B, 0, gk.MatMut.from_col_major(c1, m, n))
        gk.gemm_i8_packed_b(1, A, gk.prepack_rhs_i8(B), 0, gk.MatMut.from_col_major(c2, m, n))
        want = np.zeros(m * n, np.int32)
        oracle.gemm_i8(m, k, n, 1, a.numpy(), 1, m, b.numpy(), 1, k, 0, want, 1, m)
        assert np.array_equal(c1.cpu().numpy(), want)
        assert torch.equal(c1, c2)
        return
    B = gk.MatRef.from_row_major(bd, k, n)
    c1 = torch.zeros(m * n, dtype=tdt, device=dev)
    c2 = torch.zeros_like(c1)
    gk.gemm(1.0, A, B, 0.0, gk.MatMut.from_col_major(c1, m, n))
    gk.gemm_packed_b(1.0, A, gk.prepack_rhs(B), 0.0, gk.MatMut.from_col_major(c2, m, n))
    ints = torch.int32 if dtype == "f32" else torch.int16
    assert torch.equal(c1.view(ints), c2.view(ints))
    af = a.float().numpy() if dtype == "f32" else a.float().numpy()
    ref = oracle.gemm_f64(m, k, n, 1.0, af, 1, m, b.float().numpy(), n, 1)
    got = c1.float().cpu().numpy().reshape(n, m).T.astype(np.float64)
    if dtype == "f32":
        assert rel_frob(got, ref) <= 1e-5
    else:
        floor = 1e-3 * np.abs(ref).max()
        assert (np.abs(got - ref) <= 2.0 ** -8 * np.maximum(np.abs(ref), floor)).all()


@pytest.mark.parametrize("m,k,n", [(4, 300, 500), (16, 2048, 96), (3, 7, 40)])
def test_negative_stride_vectors(dev, m, k, n):
    """Unchecked tier: A walked backwards in both dimensions (rsa = -k, csa =
    -1 from its last element) goes straight into the skinny kernel's
    element-wise staging (tests/correctness/int8.rs:278-316 shape of test)."""
    import torch
    a = oracle.rand_i8_100(71 + m, m * k)
    b = oracle.rand_i8_100(72 + n, k * n)
    want = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a, -k, -1, b, 1, k, 0, want, n, 1, a_off=m * k - 1)
    c = torch.zeros(m * n, dtype=torch.int32, device=dev)
    gk.gemm_i8_unchecked(m, k, n, 1, to_dev(a, dev), -k, -1, to_dev(b, dev), 1, k, 0, c, n, 1,
                         a_off=m * k - 1)
    assert np.array_equal(c.cpu().numpy(), want)
