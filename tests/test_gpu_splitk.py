"""GPU parity of the split-K route: products whose 64 x 64 tile grid leaves most
CUs idle (small M*N, long K) run as partial products over K ranges plus one
reduction pass.

* i8 -> i32 and requantized outputs: bit-identical to the unsplit kernel
  (GEMMKIT_HIP_SPLITK=0 in the same process) and to the oracle -- wrapping
  i32 addition is associative, so any K partition gives the same bits.
* f32 / bf16: against the oracle's f64 closed form within the float bars of
  test_gpu_float.py; a batched call's elements stay bit-identical to
  standalone calls (the split depends on the element shape only).
"""
import os

import numpy as np
import pytest
import torch

import gemmkit_amd as gk
import oracle
from helpers import bf16_tensor_from_bits, gather, layout_strides, scatter, to_dev

pytestmark = pytest.mark.gpu


class split_off:
    """GEMMKIT_HIP_SPLITK=0 for the calls inside the block (read per call)."""

    def __enter__(self):
        self.old = os.environ.get("GEMMKIT_HIP_SPLITK")
        os.environ["GEMMKIT_HIP_SPLITK"] = "0"

    def __exit__(self, *exc):
        if self.old is None:
            del os.environ["GEMMKIT_HIP_SPLITK"]
        else:
            os.environ["GEMMKIT_HIP_SPLITK"] = self.old


@pytest.mark.parametrize("m,k,n", [(64, 2048, 2048), (17, 4096, 100), (100, 777, 300),
                                   (64, 2048, 64), (2048, 3000, 40), (90, 65536, 33)])
@pytest.mark.parametrize("lc", ["row", "col"])
@pytest.mark.parametrize("alpha,beta", [(1, 0), (3, -2)])
def test_i8_split_equals_unsplit_and_oracle(dev, m, k, n, lc, alpha, beta):
    a = oracle.rng_i8_full(11 + m, m * k)
    b = oracle.rng_i8_full(12 + n, k * n)
    rsc, csc, cl = layout_strides(m, n, lc)
    c0 = ((np.arange(cl) % 11) - 5).astype(np.int32)
    want = c0.copy()
    oracle.gemm_i8(m, k, n, alpha, a, k, 1, b, 1, k, beta, want, rsc, csc)
    ad, bd = to_dev(a, dev), to_dev(b, dev)
    outs = []
    for off in (False, True):
        cd = to_dev(c0, dev)
        call = lambda: gk.gemm_i8(alpha, gk.MatRef.from_row_major(ad, m, k),  # noqa: E731
                                  gk.MatRef(bd, k, n, 1, k), beta, gk.MatMut(cd, m, n, rsc, csc))
        if off:
            with split_off():
                call()
        else:
            call()
        outs.append(cd.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[0], want)


@pytest.mark.parametrize("axis,relu,u8", [(1, True, False), (0, False, True), (1, False, False)])
def test_requant_split_equals_unsplit(dev, axis, relu, u8):
    m, k, n = 64, 4096, 1536
    a = oracle.rng_i8_sym127(21, m * k)
    b = oracle.rng_i8_sym127(22, n * k)
    ch = n if axis else m
    u = oracle.rng_unit(23, 2 * ch)
    scales = to_dev((1e-4 + (u[:ch] + 1) / 2 * (1e-2 - 1e-4)).astype(np.float32), dev)
    bias = to_dev(np.round(u[ch:] * 65536).astype(np.int32), dev)
    ad, bd = to_dev(a, dev), to_dev(b, dev)
    req = gk.Requantize(gk.RequantScale.PerCol(scales) if axis else gk.RequantScale.PerRow(scales),
                        zero_point=7 if u8 else -3, bias=bias, bias_axis="col" if axis else "row",
                        relu=relu)
    fn = gk.gemm_i8_requant_u8 if u8 else gk.gemm_i8_requant
    outs = []
    for off in (False, True):
        cd = torch.zeros(m * n, dtype=torch.uint8 if u8 else torch.int8, device=dev)
        call = lambda: fn(gk.MatRef.from_row_major(ad, m, k), gk.MatRef(bd, k, n, 1, k),  # noqa: E731
                          req, gk.MatMut(cd, m, n, 1, m))
        if off:
            with split_off():
                call()
        else:
            call()
        outs.append(cd.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    acc = np.zeros(m * n, np.int32)
    oracle.gemm_i8(m, k, n, 1, a, k, 1, b, 1, k, 0, acc, 1, m)
    want = np.zeros(m * n, np.uint8 if u8 else np.int8)
    lo, hi = (0, 255) if u8 else (-128, 127)
    zp = 7 if u8 else -3
    if relu:
        lo = max(lo, zp)
    oracle.requant_map(m, n, acc, 1, m, 0.0, scales.cpu().numpy(), zp, bias.cpu().numpy(), axis,
                       lo, hi, want, 1, m)
    assert np.array_equal(outs[0], want)


def rel_frob(got, ref):
    return float(np.linalg.norm((got - ref).ravel()) / max(np.linalg.norm(ref.ravel()), 1e-300))


@pytest.mark.parametrize("m,k,n", [(64, 4096, 2048), (33, 1000, 129), (128, 8192, 128)])
@pytest.mark.parametrize("lc", ["row", "col"])
def test_f32_split_vs_oracle(dev, m, k, n, lc):
    a = oracle.rand_vec(31 + m, m * k).astype(np.float32)
    b = oracle.rand_vec(32 + n, k * n).astype(np.float32)
    rsc, csc, cl = layout_strides(m, n, lc)
    c0 = oracle.rand_vec(33, cl).astype(np.float32)
    ref = oracle.gemm_f64(m, k, n, 0.75, a, k, 1, b, n, 1, -1.5, c0, rsc, csc)
    cd = to_dev(c0, dev)
    gk.gemm(0.75, gk.MatRef.from_row_major(to_dev(a, dev), m, k),
            gk.MatRef.from_row_major(to_dev(b, dev), k, n), -1.5, gk.MatMut(cd, m, n, rsc, csc))
    got = gather(cd.cpu().numpy(), m, n, rsc, csc).astype(np.float64)
    assert rel_frob(got, ref) <= 1e-5


def test_bf16_out_split_vs_oracle(dev):
    m, k, n = 64, 4096, 512
    a = oracle.bf16_bits(oracle.rng_normal(41, m * k).astype(np.float32))
    b = oracle.bf16_bits(oracle.rng_normal(42, k * n).astype(np.float32))
    ref = oracle.gemm_f64(m, k, n, 1.0, oracle.bf16_to_f32(a), k, 1, oracle.bf16_to_f32(b), 1, k)
    cd = torch.zeros(m * n, dtype=torch.bfloat16, device=dev)
    gk.gemm(1.0, gk.MatRef.from_row_major(bf16_tensor_from_bits(a, dev), m, k),
            gk.MatRef(bf16_tensor_from_bits(b, dev), k, n, 1, k), 0.0,
            gk.MatMut.from_row_major(cd, m, n))
    got = cd.float().cpu().numpy().reshape(m, n).astype(np.float64)
    floor = 1e-3 * np.abs(ref).max()
    assert (np.abs(got - ref) <= 2.0 ** -8 * np.maximum(np.abs(ref), floor) + 1e-30).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_batched_split_elements_equal_standalone(dev, dtype):
    batch, m, k, n = 3, 64, 1024, 128
    g = torch.Generator(device="cpu").manual_seed(9)
    a = torch.randn(batch * m * k, generator=g).to(dtype).to(dev)
    b = torch.randn(batch * k * n, generator=g).to(dtype).to(dev)
    c = torch.zeros(batch * m * n, dtype=dtype, device=dev)
    gk.gemm_batched(batch, 1.0, gk.MatRef.from_row_major(a, m, k), m * k,
                    gk.MatRef(b, k, n, 1, k), k * n, 0.0, gk.MatMut.from_row_major(c, m, n), m * n)
    for e in range(batch):
        ce = torch.zeros(m * n, dtype=dtype, device=dev)
        gk.gemm(1.0, gk.MatRef.from_row_major(a[e * m * k:(e + 1) * m * k], m, k),
                gk.MatRef(b[e * k * n:(e + 1) * k * n], k, n, 1, k), 0.0,
                gk.MatMut.from_row_major(ce, m, n))
        ints = torch.int32 if dtype == torch.float32 else torch.int16
        assert torch.equal(ce.view(ints), c[e * m * n:(e + 1) * m * n].view(ints)), e
