"""GPU parity of the pointer-array batched forms (gemm_batched_ptr_unchecked,
gemm_batched_slice; src/api/batched.rs:711-799): every element must equal the
standalone gemm on the same inputs bit for bit, whether it runs alone or in a
run of like problems that goes out as one strided batched launch."""
import pytest
import torch

import gemmkit_amd as gk

pytestmark = pytest.mark.gpu


def randn(n, seed, dev, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, generator=g).to(dtype).to(dev)


def bits(t):
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_heterogeneous_problems_equal_standalone(dev, dtype):
    shapes = [  # m, k, n, alpha, beta, A negative row stride, C column-major
        (64, 96, 80, 1.0, 0.0, False, False),
        (300, 257, 129, 0.5, -1.0, True, False),
        (3, 5, 7, 2.0, 1.0, False, True),
        (512, 512, 512, 1.0, 0.0, False, False),
        (40, 0, 33, 1.0, 0.5, False, False),   # k == 0: C <- beta*C
        (0, 16, 16, 1.0, 0.0, False, False),   # empty
    ]
    probs, want = [], []
    for i, (m, k, n, alpha, beta, neg, ccol) in enumerate(shapes):
        a = randn(max(m * k, 1), 10 + i, dev, dtype)
        b = randn(max(k * n, 1), 20 + i, dev, dtype)
        c0 = randn(max(m * n, 1), 30 + i, dev, dtype)
        rsa, csa, a_off = (-k, 1, (m - 1) * k) if neg and m > 0 else (k, 1, 0)
        rsc, csc = (1, m) if ccol else (n, 1)
        c = c0.clone()
        ref = c0.clone()
        gk.gemm_unchecked(m, k, n, alpha, a, rsa, csa, b, n, 1, beta, ref, rsc, csc, a_off=a_off)
        probs.append(gk.GemmProblem(m, k, n, alpha, a, rsa, csa, b, n, 1, beta, c, rsc, csc,
                                    a_off=a_off))
        want.append(ref)
    gk.gemm_batched_ptr_unchecked(probs)
    for i, (p, ref) in enumerate(zip(probs, want)):
        assert torch.equal(bits(p.c), bits(ref)), i


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_run_of_like_problems_equals_standalone(dev, dtype):
    # 6 problems 128 x 256 x 192 at constant steps in shared buffers (one
    # strided batched launch), then one of another shape, then 2 more like ones
    batch, m, k, n = 6, 128, 256, 192
    a = randn(batch * m * k, 1, dev, dtype)
    b = randn(batch * k * n, 2, dev, dtype)
    c = torch.zeros(batch * m * n, dtype=dtype, device=dev)
    probs = [gk.GemmProblem(m, k, n, 1.0, a, k, 1, b, 1, k, 0.0, c, n, 1, a_off=e * m * k,
                            b_off=e * k * n, c_off=e * m * n) for e in range(batch)]
    xa, xb = randn(50 * 60, 3, dev, dtype), randn(60 * 70, 4, dev, dtype)
    xc = torch.zeros(50 * 70, dtype=dtype, device=dev)
    probs.insert(4, gk.GemmProblem(50, 60, 70, 1.0, xa, 60, 1, xb, 70, 1, 0.0, xc, 70, 1))
    gk.gemm_batched_ptr_unchecked(probs)
    for e in range(batch):
        ref = torch.zeros(m * n, dtype=dtype, device=dev)
        gk.gemm(1.0, gk.MatRef.from_row_major(a[e * m * k:(e + 1) * m * k], m, k),
                gk.MatRef(b[e * k * n:(e + 1) * k * n], k, n, 1, k), 0.0,
                gk.MatMut.from_row_major(ref, m, n))
        assert torch.equal(bits(c[e * m * n:(e + 1) * m * n]), bits(ref)), e
    ref = torch.zeros(50 * 70, dtype=dtype, device=dev)
    gk.gemm(1.0, gk.MatRef.from_row_major(xa, 50, 60), gk.MatRef.from_row_major(xb, 60, 70), 0.0,
            gk.MatMut.from_row_major(ref, 50, 70))
    assert torch.equal(bits(xc), bits(ref))


def test_slice_form_equals_standalone(dev):
    dtype = torch.bfloat16
    probs, want = [], []
    for i, (m, k, n) in enumerate([(100, 64, 80), (256, 512, 256), (7, 300, 9)]):
        a, b = randn(m * k, 40 + i, dev, dtype), randn(k * n, 50 + i, dev, dtype)
        c = torch.zeros(m * n, dtype=dtype, device=dev)
        ref = torch.zeros(m * n, dtype=dtype, device=dev)
        A, B = gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k)
        gk.gemm(0.75, A, B, 0.0, gk.MatMut.from_row_major(ref, m, n))
        probs.append(gk.BatchProblem(0.75, A, B, 0.0, gk.MatMut.from_row_major(c, m, n)))
        want.append(ref)
    gk.gemm_batched_slice(probs)
    for i, (p, ref) in enumerate(zip(probs, want)):
        assert torch.equal(bits(p.c.data), bits(ref)), i
