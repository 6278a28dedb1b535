"""Floating-point products at the benchmark's full sizes against the f64
closed form, every element (the gate elementwise: |got - ref| <= 1e-2 *
max(|ref|, 1e-3 * max|ref|), the floor because an f32 accumulation cannot
bound the relative error of an output that cancels to near zero; the
unfloored maximum is printed beside it):

  * the batched attention scores, 64 x (512 x 128) . (128 x 512) bf16 -> f32,
    B = K^T via strides, alpha = 1/sqrt(128) (src/special/batched.rs:49-141):
    all 64 elements against the oracle's f64 product, each also bit-equal to
    its standalone call (tests/batched.rs:1-3);
  * bf16 4096^3 with f32 output (the matrix-core-bound bf16 shape;
    src/kernel/mixed.rs:31-200), A row-major, B column-major;
  * bf16 4096^3 with bf16 output, a per-column bf16 bias and ReLU
    (src/kernel/mixed.rs:96-200, FusedEpi src/kernel/epilogue.rs:556-596)
    against the oracle's fused map applied to the f64 product.

The 4096^3 references are numpy's f64 matrix product of the bf16-rounded
inputs (the same closed form as the oracle's or_gemm_f64, which each test
also checks on a band of rows)."""
import numpy as np
import pytest
import torch

import gemmkit_amd as gk
import oracle
from helpers import bf16_tensor_from_bits

pytestmark = pytest.mark.gpu


def _bf16(x):
    bits = oracle.bf16_bits(x.astype(np.float32))
    return bits, oracle.bf16_to_f32(bits)


def _errors(got, ref):
    floor = 1e-3 * np.abs(ref).max()
    err = np.abs(got - ref)
    floored = float((err / np.maximum(np.abs(ref), floor)).max())
    nz = np.abs(ref) > 0
    unfloored = float((err[nz] / np.abs(ref[nz])).max()) if nz.any() else 0.0
    return floored, unfloored


def test_attention_scores_every_element(dev):
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
    worst = (0.0, 0.0)
    for z in range(Bt):
        ref = oracle.gemm_f64(S, D, S, alpha, qf[z * S * D:], D, 1, kf[z * S * D:], 1, D)
        g = got[z * S * S:(z + 1) * S * S].reshape(S, S).astype(np.float64)
        fl, unf = _errors(g, ref.reshape(S, S))
        assert fl <= 1e-2, (z, fl)
        worst = (max(worst[0], fl), max(worst[1], unf))
        if z % 8 == 5:  # a standalone call on this element, bit for bit
            one = torch.empty(S * S, dtype=torch.float32, device=dev)
            gk.gemm_bf16_f32out(alpha,
                                gk.MatRef.from_row_major(q[z * S * D:(z + 1) * S * D], S, D),
                                gk.MatRef(kk[z * S * D:(z + 1) * S * D], D, S, 1, D), 0.0,
                                gk.MatMut.from_row_major(one, S, S))
            assert np.array_equal(one.cpu().numpy().view(np.uint32),
                                  got[z * S * S:(z + 1) * S * S].view(np.uint32)), z
    print(f"attention scores 64x512x512x128, all 64 elements: max rel err floored "
          f"{worst[0]:.3g}, unfloored {worst[1]:.3g}")


def _bf16_4096(seed_a, seed_b):
    n = 4096
    abits, af = _bf16(oracle.rng_normal(seed_a, n * n))
    bbits, bf = _bf16(oracle.rng_normal(seed_b, n * n))  # B column-major: B^T row-major
    ref = af.reshape(n, n).astype(np.float64) @ bf.reshape(n, n).astype(np.float64).T
    # the closed form agrees with the oracle's f64 product on a band of rows
    band = oracle.gemm_f64(16, n, n, 1.0, af[100 * n:], n, 1, bf, 1, n)
    assert np.allclose(band.reshape(16, n), ref[100:116], rtol=1e-12, atol=1e-9)
    return abits, bbits, ref


def test_bf16_4096_f32_out_every_element(dev):
    n = 4096
    abits, bbits, ref = _bf16_4096(51, 52)
    a, b = bf16_tensor_from_bits(abits, dev), bf16_tensor_from_bits(bbits, dev)
    c = torch.empty(n * n, dtype=torch.float32, device=dev)
    gk.gemm_bf16_f32out(1.0, gk.MatRef.from_row_major(a, n, n), gk.MatRef(b, n, n, 1, n), 0.0,
                        gk.MatMut.from_row_major(c, n, n))
    got = c.cpu().numpy().reshape(n, n).astype(np.float64)
    fl, unf = _errors(got, ref)
    print(f"bf16 4096^3 -> f32: max rel err floored {fl:.3g}, unfloored {unf:.3g}")
    assert fl <= 1e-2


def test_bf16_4096_fused_bias_relu_every_element(dev):
    n = 4096
    abits, bbits, ref = _bf16_4096(53, 54)
    bias_bits, _ = _bf16(oracle.rng_normal(55, n) * 8.0)
    a, b = bf16_tensor_from_bits(abits, dev), bf16_tensor_from_bits(bbits, dev)
    bias = bf16_tensor_from_bits(bias_bits, dev)
    c = torch.empty(n * n, dtype=torch.bfloat16, device=dev)
    gk.gemm_fused(1.0, gk.MatRef.from_row_major(a, n, n), gk.MatRef(b, n, n, 1, n), 0.0,
                  gk.MatMut.from_row_major(c, n, n), gk.Bias.PerCol(bias), gk.Activation.Relu)
    got = oracle.bf16_to_f32(c.cpu().view(torch.int16).numpy().view(np.uint16)).astype(np.float64)
    # reference: the f64 product rounded once to f32 (the value a plain gemm
    # would hold before its epilogue), then the oracle's bf16 fused map
    want_bits = oracle.fused_map_bf16(ref.astype(np.float32), bias_bits, dim=1, act=1)
    want = oracle.bf16_to_f32(want_bits).astype(np.float64).ravel()
    fl, unf = _errors(got, want)
    relu_zero = int(((want == 0) != (got == 0)).sum())
    print(f"bf16 4096^3 + bias + ReLU -> bf16: max rel err floored {fl:.3g}, unfloored "
          f"{unf:.3g}; zero/non-zero pattern differs in {relu_zero} of {n * n}")
    assert fl <= 1e-2
