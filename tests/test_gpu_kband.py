"""GPU parity of the whole-row band kernel (kband_kernel in kstream.hip): short
contractions with 129..256 K bytes per row, 257..512 columns and at least one
128-row panel per CU (batch elements x row panels), e.g. the attention scores.

The kernel feeds the same matrix-core instructions the same k chunks in the
same order as the streaming kernel and the tile kernels, so every output must
equal theirs bit for bit (GEMMKIT_HIP_KBAND=0 and GEMMKIT_HIP_KSTREAM=0 in the
same process); i8 results also equal the oracle's wrapping i32 exactly and
float results stay within the f64 bars of test_gpu_float.py.  Covered: ragged
last panels and columns (waves whose 64 columns lie partly or wholly past N),
K tails inside the 256-byte row, alpha/beta with C read back, bf16 output,
row-major and padded C (the latter takes the element-wise store), batch elements
against their standalone calls (which run the streaming kernel).
"""
import os

import numpy as np
import pytest
import torch

import gemmkit_amd as gk
import oracle
from helpers import to_dev

pytestmark = pytest.mark.gpu


class env:
    def __init__(self, **kv):
        self.kv = kv

    def __enter__(self):
        self.old = {k: os.environ.get(k) for k in self.kv}
        os.environ.update(self.kv)

    def __exit__(self, *exc):
        for k, v in self.old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


def three_routes(run):
    """run() -> tensor; the band kernel's, the streaming kernel's and the tile
    kernels' results of the same call."""
    a = run().clone()
    with env(GEMMKIT_HIP_KBAND="0"):
        b = run().clone()
    with env(GEMMKIT_HIP_KSTREAM="0"):
        c = run().clone()
    return a, b, c


@pytest.mark.parametrize("batch,m,k,n", [(64, 512, 128, 512), (32, 1000, 72, 300),
                                         (40, 777, 128, 449), (256, 128, 96, 260)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.5, 1.0), (2.0, -0.75)])
def test_bf16_f32_out_equals_other_routes(dev, batch, m, k, n, alpha, beta):
    g = torch.Generator().manual_seed(batch + m + 7 * n + k)
    a = torch.randn(batch * m * k, generator=g).to(torch.bfloat16).to(dev)
    b = torch.randn(batch * n * k, generator=g).to(torch.bfloat16).to(dev)
    c0 = torch.randn(batch * m * n, generator=g).to(dev)

    def run():
        c = c0.clone()
        gk.gemm_batched_bf16_f32out(batch, alpha, gk.MatRef.from_row_major(a, m, k), m * k,
                                    gk.MatRef(b, k, n, 1, k), n * k, beta,
                                    gk.MatMut.from_row_major(c, m, n), m * n)
        return c
    s, t, u = three_routes(run)
    assert torch.equal(s, t)
    assert torch.equal(s, u)
    # element 1 (and the last) against the f64 product
    for z in (1, batch - 1):
        az = a[z * m * k:(z + 1) * m * k].double().cpu().reshape(m, k)
        bz = b[z * n * k:(z + 1) * n * k].double().cpu().reshape(n, k)
        ref = alpha * (az @ bz.T) + beta * c0[z * m * n:(z + 1) * m * n].double().cpu().reshape(m, n)
        got = s[z * m * n:(z + 1) * m * n].double().cpu().reshape(m, n)
        bar = 1e-2 * torch.maximum(ref.abs(), 1e-3 * ref.abs().max())
        assert ((got - ref).abs() <= bar).all(), z


def test_bf16_out_and_elements_equal_standalone(dev):
    batch, m, k, n = 64, 512, 128, 512
    g = torch.Generator().manual_seed(5)
    a = torch.randn(batch * m * k, generator=g).to(torch.bfloat16).to(dev)
    b = torch.randn(batch * n * k, generator=g).to(torch.bfloat16).to(dev)
    c0 = torch.randn(batch * m * n, generator=g).to(torch.bfloat16).to(dev)

    def run():
        c = c0.clone()
        gk.gemm_batched(batch, 0.5, gk.MatRef.from_row_major(a, m, k), m * k,
                        gk.MatRef(b, k, n, 1, k), n * k, 1.0,
                        gk.MatMut.from_row_major(c, m, n), m * n)
        return c
    s, t, u = three_routes(run)
    assert torch.equal(s, t)
    assert torch.equal(s, u)
    for z in (0, 29, 63):
        one = c0[z * m * n:(z + 1) * m * n].clone()
        gk.gemm(0.5, gk.MatRef.from_row_major(a[z * m * k:(z + 1) * m * k], m, k),
                gk.MatRef(b[z * n * k:(z + 1) * n * k], k, n, 1, k), 1.0,
                gk.MatMut.from_row_major(one, m, n))
        assert torch.equal(s[z * m * n:(z + 1) * m * n], one), z


@pytest.mark.parametrize("m,k,n", [(128, 64, 512), (300, 40, 300)])
def test_f32_batched_equals_other_routes(dev, m, k, n):
    batch = 256 if m <= 128 else 128
    g = torch.Generator().manual_seed(m + n)
    a = torch.randn(batch * m * k, generator=g).to(dev)
    b = torch.randn(batch * k * n, generator=g).to(dev)

    def run():
        c = torch.empty(batch * m * n, device=dev)
        gk.gemm_batched_unchecked(batch, m, k, n, 1.0, a, k, 1, m * k, b, 1, k, k * n, 0.0, c, n,
                                  1, m * n)
        return c
    s, t, u = three_routes(run)
    assert torch.equal(s, t)
    assert torch.equal(s, u)
    z = batch // 2
    ref = a[z * m * k:(z + 1) * m * k].double().cpu().reshape(m, k) @ \
        b[z * k * n:(z + 1) * k * n].double().cpu().reshape(n, k).T
    got = s[z * m * n:(z + 1) * m * n].double().cpu().reshape(m, n)
    assert ((got - ref).norm() / ref.norm()).item() <= 1e-5


@pytest.mark.parametrize("k,n,lc", [(256, 512, "row"), (200, 400, "pad"), (144, 257, "row")])
def test_i8_tall_equals_oracle_and_other_routes(dev, k, n, lc):
    """One tall product (256 panels of 128 rows) with alpha/beta, checked
    against the oracle's wrapping i32 element for element; a row stride of
    n + 1 takes the element-wise store."""
    m = 256 * 128 - 77
    a = oracle.rng_i8_full(0x901 + k, m * k)
    b = oracle.rng_i8_full(0x902 + n, k * n)  # B column-major
    rsc, csc = (n, 1) if lc == "row" else (n + 1, 1)
    c0 = ((np.arange(m * rsc) % 11) - 5).astype(np.int32)
    want = c0.copy()
    oracle.gemm_i8(m, k, n, 3, a, k, 1, b, 1, k, -2, want, rsc, csc)
    ad, bd = to_dev(a, dev), to_dev(b, dev)

    def run():
        c = to_dev(c0, dev)
        gk.gemm_i8(3, gk.MatRef.from_row_major(ad, m, k), gk.MatRef(bd, k, n, 1, k), -2,
                   gk.MatMut(c, m, n, rsc, csc))
        return c
    s, t, u = three_routes(run)
    assert torch.equal(s, t)
    assert torch.equal(s, u)
    assert np.array_equal(s.cpu().numpy(), want)
