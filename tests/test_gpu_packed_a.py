"""GPU parity of the prepacked LHS (prepack_lhs / gemm_packed_a(_fused), f32 and
bf16; src/api/packed.rs:953-1527): bit-identical to gemm / gemm_fused on the
same inputs, and the reference's checks and messages."""
import pytest
import torch

import gemmkit_amd as gk

pytestmark = pytest.mark.gpu


def randn(n, seed, dev, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, generator=g).to(dtype).to(dev)


def bits(t):
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


SHAPES = [(1, 1, 1), (5, 7, 3), (64, 128, 96), (300, 257, 129), (1024, 512, 768)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("a_col,b_col", [(False, False), (True, True)])
def test_packed_a_equals_gemm(dev, dtype, m, k, n, a_col, b_col):
    a, b = randn(m * k, 1 + m, dev, dtype), randn(k * n, 2 + n, dev, dtype)
    c0 = randn(m * n, 3, dev, dtype)
    A = gk.MatRef.from_col_major(a, m, k) if a_col else gk.MatRef.from_row_major(a, m, k)
    B = gk.MatRef.from_col_major(b, k, n) if b_col else gk.MatRef.from_row_major(b, k, n)
    want, got = c0.clone(), c0.clone()
    gk.gemm(0.5, A, B, 2.0, gk.MatMut.from_row_major(want, m, n))
    pa = gk.prepack_lhs(A)
    assert (pa.rows(), pa.cols()) == (m, k)
    gk.gemm_packed_a(0.5, pa, B, 2.0, gk.MatMut.from_row_major(got, m, n))
    assert torch.equal(bits(got), bits(want))
    # the raw form on the same handle
    raw = c0.clone()
    gk.gemm_packed_a_unchecked(0.5, pa, n, b, B.rs, B.cs, 2.0, raw, n, 1)
    assert torch.equal(bits(raw), bits(want))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("per_row,act", [(True, "relu"), (False, "leaky")])
def test_packed_a_fused_equals_gemm_fused(dev, dtype, per_row, act):
    m, k, n = 200, 300, 160
    a, b = randn(m * k, 4, dev, dtype), randn(k * n, 5, dev, dtype)
    bias_t = randn(m if per_row else n, 6, dev, dtype)
    bias = gk.Bias.PerRow(bias_t) if per_row else gk.Bias.PerCol(bias_t)
    activ = gk.Activation.Relu if act == "relu" else gk.Activation.LeakyRelu(0.125)
    A, B = gk.MatRef.from_row_major(a, m, k), gk.MatRef.from_row_major(b, k, n)
    want = torch.zeros(m * n, dtype=dtype, device=dev)
    got = torch.zeros(m * n, dtype=dtype, device=dev)
    gk.gemm_fused(1.0, A, B, 0.0, gk.MatMut.from_row_major(want, m, n), bias, activ)
    gk.gemm_packed_a_fused(1.0, gk.prepack_lhs(A), B, 0.0, gk.MatMut.from_row_major(got, m, n),
                           bias, activ)
    assert torch.equal(bits(got), bits(want))


def test_packed_a_messages(dev):
    m, k, n = 8, 16, 12
    a, b = randn(m * k, 7, dev, torch.float32), randn(k * n, 8, dev, torch.float32)
    pa = gk.prepack_lhs(gk.MatRef.from_row_major(a, m, k))
    c = torch.zeros(m * n, device=dev)
    with pytest.raises(gk.GemmkitError, match=r"^gemmkit: packed A\.cols \(16\) != B\.rows \(15\)$"):
        gk.gemm_packed_a(1.0, pa, gk.MatRef.from_row_major(b[:15 * n], 15, n), 0.0,
                         gk.MatMut.from_row_major(c, m, n))
    with pytest.raises(gk.GemmkitError, match=r"^gemmkit: packed A\.rows \(8\) != C\.rows \(7\)$"):
        gk.gemm_packed_a(1.0, pa, gk.MatRef.from_row_major(b, k, n), 0.0,
                         gk.MatMut.from_row_major(c[:7 * n], 7, n))
    with pytest.raises(gk.GemmkitError) as e:
        gk.gemm_packed_a(1.0, pa, gk.MatRef.from_row_major(b, k, n), 0.0,
                         gk.MatMut.from_col_major(c, m, n))
    assert str(e.value).endswith(
        "gemmkit: gemm_packed_a requires row-major-ish C (|csc| <= |rsc|); a column-major C "
        "would keep A in the LHS role and invalidate the prepacked LHS — use gemm() for "
        "that layout")
    buf = torch.zeros(1000, device=dev)
    with pytest.raises(gk.GemmkitError, match=r"^gemmkit: C aliases B$"):
        gk.gemm_packed_a(1.0, pa, gk.MatRef.from_row_major(buf, k, m), 0.0,
                         gk.MatMut.from_row_major(buf, m, m))
