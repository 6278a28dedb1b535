"""GPU parity of the short-contraction streaming route (kstream.hip): products
whose K fits in 256 bytes per row (K <= 128 bf16, 64 f32, 256 i8) with both
sides at least 128.

The route feeds the same matrix-core instructions the same k chunks in the
same order as the tile kernels, so every output must equal the tile route's
(GEMMKIT_HIP_KSTREAM=0 in the same process) bit for bit -- i8 also exactly
the oracle's wrapping i32, float within the float bars of test_gpu_float.py
against the f64 closed form.  Ragged edges (rows/columns past a 128 tile, K
not a multiple of 16 bytes through the pack), alpha/beta, both C layouts,
fused bias/activation, batches and the attention-score shape are covered.
"""
import os

import numpy as np
import pytest
import torch

import gemmkit_amd as gk
import oracle
from helpers import to_dev

pytestmark = pytest.mark.gpu


class kstream_off:
    def __enter__(self):
        self.old = os.environ.get("GEMMKIT_HIP_KSTREAM")
        os.environ["GEMMKIT_HIP_KSTREAM"] = "0"

    def __exit__(self, *exc):
        if self.old is None:
            del os.environ["GEMMKIT_HIP_KSTREAM"]
        else:
            os.environ["GEMMKIT_HIP_KSTREAM"] = self.old


def both_routes(run):
    """run() -> tensor; returns (streaming route, tile route)."""
    a = run().clone()
    with kstream_off():
        b = run().clone()
    return a, b


@pytest.mark.parametrize("m,k,n", [(128, 64, 128), (300, 256, 200), (512, 128, 1000),
                                   (129, 48, 257), (1000, 16, 130), (130, 7, 300)])
@pytest.mark.parametrize("lc", ["row", "col"])
def test_i8_equals_tile_route_and_oracle(dev, m, k, n, lc):
    a = oracle.rng_i8_full(0x501 + m, m * k)
    b = oracle.rng_i8_full(0x502 + n, k * n)  # B column-major
    rsc, csc = (n, 1) if lc == "row" else (1, m)
    c0 = ((np.arange(m * n) % 9) - 4).astype(np.int32)
    want = c0.copy()
    oracle.gemm_i8(m, k, n, 3, a, k, 1, b, 1, k, -2, want, rsc, csc)
    ad, bd = to_dev(a, dev), to_dev(b, dev)

    def run():
        c = to_dev(c0, dev)
        gk.gemm_i8(3, gk.MatRef.from_row_major(ad, m, k), gk.MatRef(bd, k, n, 1, k), -2,
                   gk.MatMut(c, m, n, rsc, csc))
        return c
    s, t = both_routes(run)
    assert torch.equal(s, t)
    assert np.array_equal(s.cpu().numpy(), want)


@pytest.mark.parametrize("dt,m,k,n", [(torch.float32, 256, 64, 384), (torch.float32, 300, 20, 200),
                                      (torch.bfloat16, 512, 128, 512),
                                      (torch.bfloat16, 257, 100, 129),
                                      (torch.bfloat16, 128, 8, 1024)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.5, 1.0), (2.0, -0.75)])
def test_float_equals_tile_route(dev, dt, m, k, n, alpha, beta):
    g = torch.Generator().manual_seed(m + 7 * n + k)
    a = torch.randn(m * k, generator=g).to(dt).to(dev)
    b = torch.randn(k * n, generator=g).to(dt).to(dev)
    c0 = torch.randn(m * n, generator=g).to(dt).to(dev)

    def run():
        c = c0.clone()
        gk.gemm(alpha, gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k), beta,
                gk.MatMut.from_row_major(c, m, n))
        return c
    s, t = both_routes(run)
    assert torch.equal(s, t)
    ref = alpha * (a.double().cpu().reshape(m, k) @ b.double().cpu().reshape(n, k).T) + \
        beta * c0.double().cpu().reshape(m, n)
    err = (s.double().cpu().reshape(m, n) - ref).norm() / ref.norm()
    assert err <= (1e-5 if dt == torch.float32 else 1e-2)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dim", [0, 1])
@pytest.mark.parametrize("act", ["relu", "leaky"])
def test_fused_equals_tile_route(dev, dt, dim, act):
    m, k, n = 300, 64, 260
    g = torch.Generator().manual_seed(11 + dim)
    a = torch.randn(m * k, generator=g).to(dt).to(dev)
    b = torch.randn(k * n, generator=g).to(dt).to(dev)
    bias = torch.randn(m if dim == 0 else n, generator=g).to(dt).to(dev)
    c0 = torch.randn(m * n, generator=g).to(dt).to(dev)
    bobj = gk.Bias.PerRow(bias) if dim == 0 else gk.Bias.PerCol(bias)
    aobj = gk.Activation.Relu if act == "relu" else gk.Activation.LeakyRelu(0.125)

    def run():
        c = c0.clone()
        gk.gemm_fused(0.75, gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k), 0.5,
                      gk.MatMut.from_row_major(c, m, n), bobj, aobj)
        return c
    s, t = both_routes(run)
    assert torch.equal(s, t)


def test_batched_attention_scores_equal_tile_route_and_standalone(dev):
    """64 x (512 x 512 x 128) bf16 -> f32, alpha = 1/sqrt(128), B = K^T via
    strides: the benchmark shape on both routes, and element 37 against its
    standalone call."""
    Bt, S, D = 64, 512, 128
    g = torch.Generator().manual_seed(99)
    q = torch.randn(Bt * S * D, generator=g).to(torch.bfloat16).to(dev)
    kk = torch.randn(Bt * S * D, generator=g).to(torch.bfloat16).to(dev)
    alpha = 1.0 / np.sqrt(128.0)

    def run():
        out = torch.empty(Bt * S * S, dtype=torch.float32, device=dev)
        gk.gemm_batched_bf16_f32out(Bt, alpha, gk.MatRef.from_row_major(q, S, D), S * D,
                                    gk.MatRef(kk, D, S, 1, D), S * D, 0.0,
                                    gk.MatMut.from_row_major(out, S, S), S * S)
        return out
    s, t = both_routes(run)
    assert torch.equal(s, t)
    one = torch.empty(S * S, dtype=torch.float32, device=dev)
    z = 37
    gk.gemm_bf16_f32out(alpha, gk.MatRef.from_row_major(q[z * S * D:(z + 1) * S * D], S, D),
                        gk.MatRef(kk[z * S * D:(z + 1) * S * D], D, S, 1, D), 0.0,
                        gk.MatMut.from_row_major(one, S, S))
    assert torch.equal(s[z * S * S:(z + 1) * S * S], one)
    ref = alpha * (q[z * S * D:(z + 1) * S * D].float().double().cpu().reshape(S, D) @
                   kk[z * S * D:(z + 1) * S * D].float().double().cpu().reshape(S, D).T)
    got = one.double().cpu().reshape(S, S)
    assert ((got - ref).abs() <= 1e-2 * torch.maximum(ref.abs(), 1e-3 * ref.abs().max())).all()


@pytest.mark.parametrize("batch,m,k,n", [(3, 200, 64, 300), (7, 128, 32, 128), (2, 640, 128, 256)])
def test_batched_f32_elements_equal_standalone(dev, batch, m, k, n):
    g = torch.Generator().manual_seed(batch * m + n)
    a = torch.randn(batch * m * k, generator=g).to(dev)
    b = torch.randn(batch * k * n, generator=g).to(dev)
    c = torch.empty(batch * m * n, device=dev)
    gk.gemm_batched_unchecked(batch, m, k, n, 1.0, a, k, 1, m * k, b, 1, k, k * n, 0.0, c, n, 1,
                              m * n)
    for z in range(batch):
        one = torch.empty(m * n, device=dev)
        gk.gemm_unchecked(m, k, n, 1.0, a, k, 1, b, 1, k, 0.0, one, n, 1, a_off=z * m * k,
                          b_off=z * k * n)
        assert torch.equal(c[z * m * n:(z + 1) * m * n], one), z
