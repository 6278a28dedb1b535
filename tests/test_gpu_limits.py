"""GPU parity at the edges of the input space the reference accepts.

gemmkit takes any usize shape and batch and any isize strides on its unchecked
tier (src/api.rs:469-580, src/api/batched.rs:594-711), failing closed only
where a size computation overflows (src/workspace.rs:25-45).  These cases run
through pieces the device kernels address: negative row strides (packed,
tests/correctness/int8.rs:278-316), negative batch strides, batches beyond one
launch's grid, row strides and K beyond the kernels' 32-bit row offsets (K is
sliced and summed as the reference's kc slices are, src/driver.rs:725-730),
batched split-K products with bounded partial-sum memory, batched skinny
products in one launch, and a workspace that must not grow under HIP graph
capture.  i8 results are bit-exact against the oracle; float results are
bit-equal to the standalone call where the reference promises it
(tests/batched.rs:1-3), else within the float bar of test_gpu_float.py.
"""
import numpy as np
import pytest
import torch

import gemmkit_amd as gk
import oracle
from helpers import to_dev

pytestmark = pytest.mark.gpu


def i8_oracle(m, k, n, a, rsa, csa, b, rsb, csb, a_off=0, b_off=0):
    want = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a[a_off:], rsa, csa, b[b_off:], rsb, csb, 0, want, n, 1)
    return want


@pytest.mark.parametrize("m,k,n", [(12, 64, 7), (12, 64, 300), (300, 128, 257), (4, 256, 3000)])
def test_negative_aligned_row_stride_a(dev, m, k, n):
    """A based at its last row with rsa = -k, a multiple of 16 bytes: the kernels
    address rows with unsigned 32-bit offsets, so the host must pack it."""
    a = oracle.rand_i8_100(0x51 + m, m * k)
    b = oracle.rand_i8_100(0x52 + n, k * n)
    # logical A row i is stored at row m-1-i
    a_rev = a.reshape(m, k)[::-1].ravel().copy()
    want = i8_oracle(m, k, n, a, k, 1, b, 1, k)
    c = torch.zeros(m * n, dtype=torch.int32, device=dev)
    gk.gemm_i8_unchecked(m, k, n, 1, to_dev(a_rev, dev), -k, 1, to_dev(b, dev), 1, k, 0, c, n, 1,
                         a_off=(m - 1) * k)
    assert np.array_equal(c.cpu().numpy(), want)


@pytest.mark.parametrize("m,k,n", [(4, 256, 3000), (300, 128, 257), (9, 64, 20)])
def test_negative_aligned_column_stride_b(dev, m, k, n):
    """B column-major with its columns in reverse order (csb = -k): B^T has a
    negative row stride on the skinny (m <= 16) and tile routes."""
    a = oracle.rand_i8_100(0x61 + m, m * k)
    b = oracle.rand_i8_100(0x62 + n, k * n)  # column j of B at b[j*k:(j+1)*k]
    b_rev = b.reshape(n, k)[::-1].ravel().copy()
    want = i8_oracle(m, k, n, a, k, 1, b, 1, k)
    c = torch.zeros(m * n, dtype=torch.int32, device=dev)
    gk.gemm_i8_unchecked(m, k, n, 1, to_dev(a, dev), k, 1, to_dev(b_rev, dev), 1, -k, 0, c, n, 1,
                         b_off=(n - 1) * k)
    assert np.array_equal(c.cpu().numpy(), want)


@pytest.mark.parametrize("m,k,n", [(33, 64, 40), (3, 512, 700), (300, 96, 260)])
def test_negative_batch_stride(dev, m, k, n):
    """Batch element z of A at base - z*a_bs: each element equals its
    standalone call bit for bit."""
    batch = 3
    g = torch.Generator().manual_seed(m + n)
    a = torch.randn(batch * m * k, generator=g).to(dev)
    b = torch.randn(batch * k * n, generator=g).to(dev)
    c = torch.empty(batch * m * n, device=dev)
    gk.gemm_batched_unchecked(batch, m, k, n, 1.0, a, k, 1, -m * k, b, n, 1, k * n, 0.0, c, n, 1,
                              m * n, a_off=(batch - 1) * m * k)
    for z in range(batch):
        one = torch.empty(m * n, device=dev)
        gk.gemm_unchecked(m, k, n, 1.0, a, k, 1, b, n, 1, 0.0, one, n, 1,
                          a_off=(batch - 1 - z) * m * k, b_off=z * k * n)
        assert torch.equal(c[z * m * n:(z + 1) * m * n], one), z


@pytest.mark.parametrize("m,k,n,a_bs", [(2, 1024, 700, 2 * 1024 + 1), (3, 1536, 900, 3 * 1536 + 3),
                                        (1, 2048, 500, 2049)])
def test_vector_route_independent_of_alignment(dev, m, k, n, a_bs):
    """f32 with 2..4 vectors and 4..8 KiB rows takes the wavefront GEMV; an odd
    batch stride (unaligned elements) must not move a batched element to
    another kernel, which would sum in another order."""
    batch = 3
    g = torch.Generator().manual_seed(7 * m + n)
    a = torch.randn((batch - 1) * a_bs + m * k, generator=g).to(dev)
    b = torch.randn(k * n, generator=g).to(dev)
    c = torch.empty(batch * m * n, device=dev)
    gk.gemm_batched_unchecked(batch, m, k, n, 1.0, a, k, 1, a_bs, b, 1, k, 0, 0.0, c, n, 1, m * n)
    for z in range(batch):
        one = torch.empty(m * n, device=dev)
        gk.gemm_unchecked(m, k, n, 1.0, a, k, 1, b, 1, k, 0.0, one, n, 1, a_off=z * a_bs)
        assert torch.equal(c[z * m * n:(z + 1) * m * n], one), z


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,k,n", [(4, 512, 3000), (1, 700, 2000), (16, 256, 1000),
                                   (3000, 512, 6)])
def test_batched_vector_route_one_launch(dev, dt, m, k, n):
    """The skinny and GEMV kernels take the whole batch in one launch (grid y);
    every element equals its standalone call bit for bit."""
    batch = 5
    g = torch.Generator().manual_seed(m * 31 + n)
    a = torch.randn(batch * m * k, generator=g).to(dt).to(dev)
    b = torch.randn(batch * k * n, generator=g).to(dt).to(dev)
    c = torch.empty(batch * m * n, dtype=dt, device=dev)
    gk.gemm_batched_unchecked(batch, m, k, n, 1.0, a, k, 1, m * k, b, 1, k, k * n, 0.0, c, n, 1,
                              m * n)
    for z in range(batch):
        one = torch.empty(m * n, dtype=dt, device=dev)
        gk.gemm_unchecked(m, k, n, 1.0, a, k, 1, b, 1, k, 0.0, one, n, 1, a_off=z * m * k,
                          b_off=z * k * n)
        assert torch.equal(c[z * m * n:(z + 1) * m * n], one), z


def test_batched_split_k_bounded_workspace(dev, monkeypatch):
    """A batch of small, long-K f32 products keeps its per-element split (bit
    equality with the standalone call) but runs through a bounded partial-sum
    slab: 300 elements of 64x64x4096 would need 300 x 32 x 16 KiB = 150 MiB of
    slabs at once.  (Split K forced: by default this shape takes the small f32
    route, which needs no workspace.)"""
    monkeypatch.setenv("GEMMKIT_HIP_SMALLF32", "0")
    batch, m, k, n = 300, 64, 4096, 64
    g = torch.Generator().manual_seed(5)
    a = torch.randn(batch * m * k, generator=g).to(dev)
    b = torch.randn(batch * k * n, generator=g).to(dev)
    c = torch.empty(batch * m * n, device=dev)
    ws = gk.Workspace()
    gk.gemm_batched_unchecked(batch, m, k, n, 1.0, a, k, 1, m * k, b, 1, k, k * n, 0.0, c, n, 1,
                              m * n, ws=ws)
    assert 0 < ws.bytes() <= (64 << 20) + (1 << 20)
    for z in (0, 1, 150, 299):
        one = torch.empty(m * n, device=dev)
        gk.gemm_unchecked(m, k, n, 1.0, a, k, 1, b, 1, k, 0.0, one, n, 1, a_off=z * m * k,
                          b_off=z * k * n)
        assert torch.equal(c[z * m * n:(z + 1) * m * n], one), z
    # the f64 closed form on one element
    az = a[150 * m * k:151 * m * k].double().cpu().reshape(m, k)
    bz = b[150 * k * n:151 * k * n].double().cpu().reshape(n, k).T
    ref = (az @ bz).numpy()
    got = c[150 * m * n:151 * m * n].double().cpu().numpy().reshape(m, n)
    assert np.linalg.norm(got - ref) <= 1e-5 * np.linalg.norm(ref)


@pytest.mark.parametrize("m,k,n", [(20, 16, 20), (3, 8, 5)])
def test_batch_beyond_one_grid(dev, m, k, n):
    """65537 batch elements (two more than one launch's grid takes): the tile
    route (short side 20) and the skinny route (short side 3), on small
    integers, bit-exact against the exact product."""
    batch = 65537
    a = oracle.rand_i8_100(0x71 + m, batch * m * k)
    b = oracle.rand_i8_100(0x72 + n, batch * k * n)
    A = a.reshape(batch, m, k).astype(np.int64)
    B = b.reshape(batch, n, k).astype(np.int64)  # B column-major per element
    want = np.einsum("zik,zjk->zij", A, B).astype(np.int32).ravel()
    # gemm_batched has no i8 form; the f32 entry on these small integers is
    # exact (every partial sum is an integer below 2^24)
    ad = to_dev(a.astype(np.float32), dev)
    bd = to_dev(b.astype(np.float32), dev)
    c = torch.empty(batch * m * n, device=dev)
    gk.gemm_batched_unchecked(batch, m, k, n, 1.0, ad, k, 1, m * k, bd, 1, k, k * n, 0.0, c, n, 1,
                              m * n)
    assert np.array_equal(c.cpu().numpy().astype(np.int64), want.astype(np.int64))


def test_row_stride_beyond_32bit_offsets(dev):
    """A row stride of 12 MB (3M f32) is legal; the tile kernels address 256
    rows with 32-bit offsets, so the operand is packed first."""
    m, k, n = 40, 64, 48
    rsa = 3 * 1024 * 1024
    g = torch.Generator().manual_seed(11)
    a = torch.zeros((m - 1) * rsa + k, device=dev)
    rows = torch.randn(m, k, generator=g)
    for i in range(m):
        a[i * rsa:i * rsa + k] = rows[i].to(dev)
    b = torch.randn(k * n, generator=g).to(dev)
    c = torch.empty(m * n, device=dev)
    gk.gemm_unchecked(m, k, n, 1.0, a, rsa, 1, b, n, 1, 0.0, c, n, 1)
    ref = rows.double() @ b.double().cpu().reshape(k, n)
    got = c.double().cpu().reshape(m, n)
    assert torch.linalg.norm(got - ref) <= 1e-5 * torch.linalg.norm(ref)


LONG_K = (1 << 23) + 80  # 8 MiB + 80 bytes of i8: beyond one launch's 32-bit row offsets


def _exact_i8(m, n, a, b):
    """Exact i32 of A (m x K, row-major) times B given as n x K rows: f64 BLAS
    over 1M-wide K blocks (every partial sum is an integer below 2^53)."""
    A, B = a.reshape(m, -1), b.reshape(n, -1)
    out = np.zeros((m, n), np.float64)
    for p0 in range(0, A.shape[1], 1 << 20):
        out += A[:, p0:p0 + (1 << 20)].astype(np.float64) @ \
            B[:, p0:p0 + (1 << 20)].astype(np.float64).T
    return out


@pytest.mark.parametrize("m,n", [(24, 24), (1, 64), (12, 40)])
def test_long_k_i8(dev, m, n):
    """K = 2^23 + 80 int8: the tile route (24 x 24) runs K slices summed in an
    i32 slab; the GEMV (one vector) and skinny (12) routes take it whole or
    sliced -- all bit-exact."""
    k = LONG_K
    a = oracle.rng_i8_full(0x81 + m, m * k)
    b = oracle.rng_i8_full(0x82 + n, n * k)  # B column-major
    want = _exact_i8(m, n, a, b)
    assert np.abs(want).max() < 2**31
    c = torch.zeros(m * n, dtype=torch.int32, device=dev)
    gk.gemm_i8_unchecked(m, k, n, 1, to_dev(a, dev), k, 1, to_dev(b, dev), 1, k, 0, c, n, 1)
    assert np.array_equal(c.cpu().numpy(), want.astype(np.int32).ravel())


def test_long_k_requant(dev):
    """The K-sliced route applies requantization once, to the summed i32."""
    m, n, k = 20, 18, LONG_K
    a = oracle.rng_i8_full(0x91, m * k)
    b = oracle.rng_i8_full(0x92, n * k)
    acc = _exact_i8(m, n, a, b).astype(np.int64)
    assert np.abs(acc).max() < 2**31
    acc = acc.astype(np.int32).ravel()
    scales = np.linspace(1e-5, 3e-4, m).astype(np.float32)
    bias = (np.arange(m, dtype=np.int32) * 1000 - 7000).astype(np.int32)
    want = np.zeros(m * n, np.int8)
    oracle.requant_map(m, n, acc, n, 1, 0.0, scales, 2, bias, 0, -128, 127, want, n, 1)
    q = torch.zeros(m * n, dtype=torch.int8, device=dev)
    req = gk.Requantize(gk.RequantScale.PerRow(to_dev(scales, dev)), 2, to_dev(bias, dev))
    gk.gemm_i8_requant(gk.MatRef.from_row_major(to_dev(a, dev), m, k),
                       gk.MatRef(to_dev(b, dev), k, n, 1, k), req,
                       gk.MatMut.from_row_major(q, m, n))
    assert np.array_equal(q.cpu().numpy(), want)


def test_long_k_f32(dev):
    """K = 2^21 + 20 f32 (8 MiB + 80 bytes per row) on the tile route: the
    slices accumulate in f32 as the reference's kc slices do; rel-Frobenius
    against the f64 product."""
    m, n, k = 20, 24, (1 << 21) + 20
    g = torch.Generator().manual_seed(3)
    a = torch.randn(m * k, generator=g)
    b = torch.randn(n * k, generator=g)
    ref = a.double().reshape(m, k) @ b.double().reshape(n, k).T
    c = torch.empty(m * n, device=dev)
    gk.gemm_unchecked(m, k, n, 1.0, a.to(dev), k, 1, b.to(dev), 1, k, 0.0, c, n, 1)
    got = c.double().cpu().reshape(m, n)
    assert torch.linalg.norm(got - ref) <= 1e-5 * torch.linalg.norm(ref)


def test_capture_needs_a_sized_workspace(dev):
    """Under HIP graph capture a call that would grow its workspace fails with a
    clear error instead of allocating; a workspace sized beforehand
    (Workspace::with_capacity, src/workspace.rs:78) captures and replays."""
    m, k, n = 256, 192, 320
    a = oracle.rand_i8_100(0xA1, m * k)
    b = oracle.rand_i8_100(0xA2, k * n)  # B row-major: packed into the workspace
    want = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a, k, 1, b, n, 1, 0, want, n, 1)
    ad, bd = to_dev(a, dev), to_dev(b, dev)
    c = torch.zeros(m * n, dtype=torch.int32, device=dev)
    A, B, C = gk.MatRef.from_row_major(ad, m, k), gk.MatRef.from_row_major(bd, k, n), \
        gk.MatMut.from_row_major(c, m, n)
    gk.set_synchronous(False)
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        empty = gk.Workspace()
        err = None
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                try:
                    gk.gemm_i8(1, A, B, 0, C, ws=empty)
                except gk.GemmkitError as e:
                    err = str(e)
        assert err is not None and "graph capture" in err, err
        assert empty.bytes() == 0
        sized = gk.Workspace.with_capacity(1 << 20)
        assert sized.bytes() >= 1 << 20
        graph2 = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph2, stream=side):
                gk.gemm_i8(1, A, B, 0, C, ws=sized)
        torch.cuda.current_stream().wait_stream(side)
        for _ in range(3):
            c.zero_()
            torch.cuda.synchronize()
            graph2.replay()
            torch.cuda.synchronize()
            assert np.array_equal(c.cpu().numpy(), want)
    finally:
        gk.set_synchronous(True)
