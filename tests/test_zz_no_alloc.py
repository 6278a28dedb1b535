"""GPU parity of gk_gemm_i8_unchecked_noalloc, the no-allocation twin of
gk_gemm_i8_unchecked (no counterpart in the reference): called through the C
ABI, its output must equal the allocating entry point's bit for bit (and the
oracle's), on consecutive calls that reuse the static scratch -- the second
with a smaller input -- and on shapes that need scratch (a packed operand, the
split-K partial sums).  A product that needs more than the scratch holds fails
with GK_ERR_NOMEM before launching anything.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
from gemmkit_amd import _lib
from helpers import to_dev

pytestmark = pytest.mark.gpu

GK_ERR_NOMEM = -8


def run_pair(dev, m, k, n, la, lb, seed):
    """Both entry points on the same inputs; returns (noalloc C, allocating C,
    oracle C).  la/lb: 'row' or 'col' layouts of A and B; C row-major."""
    L = _lib.lib()
    a = oracle.rng_i8_full(seed, m * k)
    b = oracle.rng_i8_full(seed + 1, k * n)
    rsa, csa = (k, 1) if la == "row" else (1, m)
    rsb, csb = (n, 1) if lb == "row" else (1, k)
    ad, bd = to_dev(a, dev), to_dev(b, dev)
    c0 = ((np.arange(m * n) % 5) - 2).astype(np.int32)
    outs = []
    for name in ("gk_gemm_i8_unchecked_noalloc", "gk_gemm_i8_unchecked"):
        cd = to_dev(c0, dev)
        args = (m, k, n, 3, ad.data_ptr(), rsa, csa, bd.data_ptr(), rsb, csb, -2, cd.data_ptr(),
                n, 1, 1)
        fn = getattr(L, name)
        rc = fn(*args) if name.endswith("noalloc") else fn(None, *args)
        assert rc == 0, (name, rc, _lib.last_error())
        torch.cuda.synchronize()
        outs.append(cd.cpu().numpy())
    want = c0.copy()
    oracle.gemm_i8(m, k, n, 3, a, rsa, csa, b, rsb, csb, -2, want, n, 1)
    return outs[0], outs[1], want


def test_noalloc_equals_allocating_entry_two_calls():
    dev = torch.device("cuda:0")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    # 1: both operands packed into the scratch (A column-major, B row-major)
    got, ref, want = run_pair(dev, 1024, 2048, 768, "col", "row", 0x1001)
    assert np.array_equal(got, ref) and np.array_equal(got, want)
    # 2: smaller, split K (96 x 80 output, K = 8192) with a packed B: the
    # partial sums land where call 1 left its packed operands
    got, ref, want = run_pair(dev, 96, 8192, 80, "row", "row", 0x2002)
    assert np.array_equal(got, ref) and np.array_equal(got, want)


def test_noalloc_rejects_products_beyond_its_scratch():
    dev = torch.device("cuda:0")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    L = _lib.lib()
    # B row-major 8192 x 8192 would pack to 64 MiB of B^T alone; nothing is
    # read or written before the check, so small placeholder buffers serve.
    a = torch.zeros(16, dtype=torch.int8, device=dev)
    c = torch.zeros(16, dtype=torch.int32, device=dev)
    m = k = n = 8192
    rc = L.gk_gemm_i8_unchecked_noalloc(m, k, n, 1, a.data_ptr(), 1, m, a.data_ptr(), n, 1, 0,
                                         c.data_ptr(), n, 1, 1)
    assert rc == GK_ERR_NOMEM
    assert "scratch" in _lib.last_error()
