"""GPU parity of the matrix-vector kernels under every launch shape the tuning
switches select (GEMMKIT_HIP_GEMV_SHAPE="rows,wgs" for the wavefront GEMV,
GEMMKIT_HIP_SKINNY_SHAPE="rows,wgs" for the matrix-core skinny kernel).

The launch shape changes how rows are dealt out to waves and workgroups, not
what a row's sum is: i8 outputs stay bit-exact against the oracle under every
shape, and the skinny kernel's float outputs are identical to its default
shape's (each row's K ranges and their summation order depend on K only).
"""
import os

import pytest
import torch

import gemmkit_amd as gk
from test_gpu_i8 import run_case

pytestmark = pytest.mark.gpu


class env:
    def __init__(self, name, value):
        self.name, self.value = name, value

    def __enter__(self):
        self.old = os.environ.get(self.name)
        os.environ[self.name] = self.value

    def __exit__(self, *exc):
        if self.old is None:
            del os.environ[self.name]
        else:
            os.environ[self.name] = self.old


# one vector: 4 KiB rows (2 rows per wave iteration by default), 1 KiB rows
# (4 per iteration), the vector on either side, ragged row counts
GEMV_SHAPES = [(1, 4096, 3001), (1, 1024, 2049), (2001, 2048, 1), (1, 8192, 257)]


@pytest.mark.parametrize("m,k,n", GEMV_SHAPES)
@pytest.mark.parametrize("rows", [1, 2, 4])
@pytest.mark.parametrize("wgs", [1, 3, 8])
def test_i8_gemv_launch_shapes(dev, m, k, n, rows, wgs):
    with env("GEMMKIT_HIP_GEMV_SHAPE", f"{rows},{wgs}"):
        run_case(dev, m, k, n, 3, -2, "row", "col", "row", seed=rows * 10 + wgs)


SKINNY_SHAPES = [(8, 4096, 3001), (5, 1040, 777), (300, 4112, 16), (16, 64, 100)]


@pytest.mark.parametrize("m,k,n", SKINNY_SHAPES)
@pytest.mark.parametrize("rows", [8, 16, 32])
@pytest.mark.parametrize("wgs", [1, 2, 4])
def test_i8_skinny_launch_shapes(dev, m, k, n, rows, wgs):
    with env("GEMMKIT_HIP_SKINNY_SHAPE", f"{rows},{wgs}"):
        run_case(dev, m, k, n, 3, -2, "row", "col", "row", seed=rows + wgs)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_float_skinny_launch_shapes_identical(dev, dt):
    m, k, n = 8, 2000, 1500
    g = torch.Generator().manual_seed(5)
    a = torch.randn(m * k, generator=g).to(dt).to(dev)
    b = torch.randn(k * n, generator=g).to(dt).to(dev)

    def run():
        c = torch.empty(m * n, dtype=torch.float32, device=dev)
        if dt == torch.float32:
            gk.gemm(1.0, gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k), 0.0,
                    gk.MatMut.from_row_major(c, m, n))
        else:
            gk.gemm_bf16_f32out(1.0, gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k),
                                0.0, gk.MatMut.from_row_major(c, m, n))
        return c
    base = run()
    for rows in (8, 16, 32):
        for wgs in (1, 2, 4):
            with env("GEMMKIT_HIP_SKINNY_SHAPE", f"{rows},{wgs}"):
                assert torch.equal(run(), base), (rows, wgs)
    ref = a.double().cpu().reshape(m, k) @ b.double().cpu().reshape(n, k).T
    err = (base.double().cpu().reshape(m, n) - ref).norm() / ref.norm()
    assert err <= (1e-5 if dt == torch.float32 else 1e-2)
