"""GPU parity of the small f32 route (small.hip): f32 products whose 64 x 64
tiles leave most CUs idle and whose K would otherwise be split (gemmkit's f32
512^3, all row-major, is the shape it serves).  One launch reads the operands
in place with any strides and adds the sixteen waves' K ranges in wave order.

Bars: the float suite's (relative Frobenius <= 1e-5 and the reference's own
8*k*eps gate against the f64 product); batched elements bit-identical to
standalone calls; alpha/beta and both C orientations; ragged blocks and K;
and the split-K route (GEMMKIT_HIP_SMALLF32=0) agreeing within the same bar.
"""
import os

import numpy as np
import pytest
import torch

import gemmkit_amd as gk
import oracle
from helpers import gather, layout_strides, scatter, to_dev
from test_gpu_float import F32_EPS, rel_frob

pytestmark = pytest.mark.gpu


class small_off:
    def __enter__(self):
        self.old = os.environ.get("GEMMKIT_HIP_SMALLF32")
        os.environ["GEMMKIT_HIP_SMALLF32"] = "0"

    def __exit__(self, *exc):
        if self.old is None:
            del os.environ["GEMMKIT_HIP_SMALLF32"]
        else:
            os.environ["GEMMKIT_HIP_SMALLF32"] = self.old


def _case(dev, m, k, n, la, lb, lc, alpha, beta, seed):
    a = oracle.rand_vec(seed, m * k).astype(np.float32).reshape(m, k)
    b = oracle.rand_vec(seed + 1, k * n).astype(np.float32).reshape(k, n)
    c0 = oracle.rand_vec(seed + 2, m * n).astype(np.float32).reshape(m, n)
    rsa, csa, al = layout_strides(m, k, la, 3)
    rsb, csb, bl = layout_strides(k, n, lb, 3)
    rsc, csc, cl = layout_strides(m, n, lc, 3)
    abuf, bbuf, cbuf = scatter(a, rsa, csa, al), scatter(b, rsb, csb, bl), scatter(c0, rsc, csc, cl)
    ref = oracle.gemm_f64(m, k, n, alpha, abuf, rsa, csa, bbuf, rsb, csb, beta, cbuf, rsc, csc)

    def run():
        cd = to_dev(cbuf, dev)
        gk.gemm(alpha, gk.MatRef(to_dev(abuf, dev), m, k, rsa, csa),
                gk.MatRef(to_dev(bbuf, dev), k, n, rsb, csb), beta, gk.MatMut(cd, m, n, rsc, csc))
        return gather(cd.cpu().numpy(), m, n, rsc, csc).astype(np.float64)
    got = run()
    assert rel_frob(got, ref) <= 1e-5
    num = np.linalg.norm((got - ref).ravel())
    den = np.linalg.norm(a.ravel()) * np.linalg.norm(b.ravel()) * abs(alpha) + \
        abs(beta) * np.linalg.norm(c0.ravel()) + 1e-30
    assert num / den <= 8 * k * F32_EPS
    with small_off():
        other = run()
    assert rel_frob(other, ref) <= 1e-5
    return got


def test_config_512_all_row_major(dev):
    _case(dev, 512, 512, 512, "row", "row", "row", 1.0, 0.0, 0x5120)


@pytest.mark.parametrize("m,k,n", [(100, 700, 200), (33, 129, 65), (257, 1000, 31 + 64),
                                   (64, 2048, 64), (480, 300, 500), (256, 8192, 256),
                                   (200, 4001, 100)])
@pytest.mark.parametrize("la,lb,lc", [("row", "row", "row"), ("col", "col", "col"),
                                      ("row+", "col+", "row+"), ("col", "row", "col+")])
def test_layouts_and_ragged(dev, m, k, n, la, lb, lc):
    _case(dev, m, k, n, la, lb, lc, 0.75, -1.25, m + 3 * k + 7 * n)


def test_batched_elements_equal_standalone(dev):
    batch, m, k, n = 5, 200, 600, 300
    g = torch.Generator().manual_seed(77)
    a = torch.randn(batch * m * k, generator=g).to(dev)
    b = torch.randn(batch * k * n, generator=g).to(dev)  # row-major k x n per element
    c = torch.empty(batch * m * n, device=dev)
    gk.gemm_batched_unchecked(batch, m, k, n, 1.0, a, k, 1, m * k, b, n, 1, k * n, 0.0, c, n, 1,
                              m * n)
    for z in range(batch):
        one = torch.empty(m * n, device=dev)
        gk.gemm_unchecked(m, k, n, 1.0, a, k, 1, b, n, 1, 0.0, one, n, 1, a_off=z * m * k,
                          b_off=z * k * n)
        assert torch.equal(c[z * m * n:(z + 1) * m * n], one), z


def test_negative_strides(dev):
    """The unchecked tier's negative strides: A with reversed rows, B with
    reversed columns, read in place."""
    m, k, n = 96, 256, 160
    g = torch.Generator().manual_seed(78)
    a = torch.randn(m * k, generator=g).to(dev)
    b = torch.randn(k * n, generator=g).to(dev)
    c = torch.empty(m * n, device=dev)
    # A(i, p) = a[(m-1-i)*k + p], B(p, j) = b[p*n + (n-1-j)]
    gk.gemm_unchecked(m, k, n, 1.0, a, -k, 1, b, n, -1, 0.0, c, n, 1, a_off=(m - 1) * k,
                      b_off=n - 1)
    A = a.cpu().double().reshape(m, k).flip(0)
    B = b.cpu().double().reshape(k, n).flip(1)
    ref = A @ B
    got = c.cpu().double().reshape(m, n)
    assert ((got - ref).norm() / ref.norm()).item() <= 1e-5
