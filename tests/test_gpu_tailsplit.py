"""GPU parity of the multi-round plans: products whose 256-wide tiles take
two rounds of the CUs with a short last round run either as one round of
256 x 352 strip tiles (int8) or 256 x 384 tiles (bf16, or a pitch past 352)
at a column pitch (the default where the model takes it: the layer shapes;
both tiles are also forced here with GEMMKIT_HIP_TILE) or, with that plan off (GEMMKIT_HIP_WIDE=0), as a tail
split into two launches (the full rounds' columns with the chosen tile, the
rest with smaller tiles at a column pitch that makes the rest one round).
Every output element keeps its K order, so all five plans must equal the
single launch (both off) bit for bit, for every epilogue: alpha/beta,
requantization with per-column and per-row channels, fused bias and ReLU, and
the orientation swap of a column-major C."""
import os

import pytest
import torch

import gemmkit_amd as gk

pytestmark = pytest.mark.gpu

_SWITCHES = ("GEMMKIT_HIP_WIDE", "GEMMKIT_HIP_TAILSPLIT", "GEMMKIT_HIP_TILE")


class env:
    """Sets the plan switches to `values` (others unset) for a block."""

    def __init__(self, **values):
        self.values = values

    def __enter__(self):
        self.old = {k: os.environ.get(k) for k in _SWITCHES}
        for k in _SWITCHES:
            os.environ.pop(k, None)
        os.environ.update(self.values)

    def __exit__(self, *exc):
        for k, v in self.old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


DEFAULT = {}
WIDE384 = {"GEMMKIT_HIP_TILE": "256x384w8k128"}
STRIP352 = {"GEMMKIT_HIP_TILE": "256x352w8k128"}
STRIP352M16 = {"GEMMKIT_HIP_TILE": "256x352w8m16"}  # int8 only
SPLIT = {"GEMMKIT_HIP_WIDE": "0"}
SINGLE = {"GEMMKIT_HIP_WIDE": "0", "GEMMKIT_HIP_TAILSPLIT": "0"}


def plans(plan_args, wide=True):
    """The plan under each setting; asserts the tail split is taken with the
    wide plan off, and (wide=True) the one-round plan by default: 256 x 352
    tiles on 16x16 MFMAs for int8, 256 x 384 tiles for bf16."""
    with env(**SPLIT):
        assert gk.debug_plan(*plan_args)[1] > 0
    if wide:
        with env(**DEFAULT):
            want = "256x352w8m16" if plan_args[0] == "i8" else "256x384w8k128"
            assert gk.debug_plan(*plan_args)[0] == want


def both(call, i8=False):
    """Runs call() under the default plan, the forced 256 x 384 and 256 x 352
    tiles (and, i8, the 256 x 352 tile on 16x16 MFMAs), the tail split and the
    single launch; returns (default, 384, 352[, 352 m16], split, single)."""
    out = []
    for e in (DEFAULT, WIDE384, STRIP352) + ((STRIP352M16,) if i8 else ()) + (SPLIT, SINGLE):
        with env(**e):
            out.append(call())
    return out


def bits(t):
    return t.view(torch.int8 if t.element_size() == 1 else
                  torch.int16 if t.element_size() == 2 else torch.int32)


def rand_i8(n, seed, dev, lo=-128):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, 128, (n,), dtype=torch.int8, generator=g).to(dev)


@pytest.mark.parametrize("c_col_major", [False, True])
def test_i8_alpha_beta(dev, c_col_major):
    m, k, n = 2048, 4096, 11008
    if c_col_major:
        m, n = n, m  # kernel frame: M = 2048, N = 11008 after the swap
    plans(("i8", "i32", 2048, 11008, k))
    a, b = rand_i8(m * k, 1, dev), rand_i8(k * n, 2, dev)
    g = torch.Generator().manual_seed(3)
    c0 = torch.randint(-1000, 1000, (m * n,), dtype=torch.int32, generator=g).to(dev)
    C = (lambda t: gk.MatMut.from_col_major(t, m, n)) if c_col_major else \
        (lambda t: gk.MatMut.from_row_major(t, m, n))

    def call():
        c = c0.clone()
        gk.gemm_i8(3, gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k), -2, C(c))
        return c
    *plans_out, single = both(call, i8=True)
    for o in plans_out:
        assert torch.equal(o, single)


@pytest.mark.parametrize("axis,u8", [(1, False), (0, True)])
def test_requant(dev, axis, u8):
    m, k, n = 2048, 4096, 11008
    plans(("i8", "q8", m, n, k))
    a, b = rand_i8(m * k, 4, dev, -127), rand_i8(n * k, 5, dev, -127)
    ch = n if axis else m
    g = torch.Generator().manual_seed(6)
    scales = (1e-4 + torch.rand(ch, generator=g) * (1e-2 - 1e-4)).to(dev)
    bias = torch.randint(-65536, 65537, (ch,), dtype=torch.int32, generator=g).to(dev)
    req = gk.Requantize(gk.RequantScale.PerCol(scales) if axis else gk.RequantScale.PerRow(scales),
                        zero_point=7 if u8 else -3, bias=bias, bias_axis="col" if axis else "row",
                        relu=True)
    fn = gk.gemm_i8_requant_u8 if u8 else gk.gemm_i8_requant

    def call():
        c = torch.zeros(m * n, dtype=torch.uint8 if u8 else torch.int8, device=dev)
        fn(gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k), req,
           gk.MatMut.from_row_major(c, m, n))
        return c
    *plans_out, single = both(call, i8=True)
    for o in plans_out:
        assert torch.equal(o, single)


def test_bf16_fused_bias_relu(dev):
    """bf16: the one-round plans and the tail split sum in the 32x32 tiles'
    order (bit-identical); the single launch takes the 16x16-MFMA tile,
    which sums 32 k per instruction, so it agrees within the bf16 bars."""
    m, k, n = 2048, 4096, 11008
    plans(("bf16", "bf16", m, n, 2 * k))
    g = torch.Generator().manual_seed(7)
    a = torch.randn(m * k, generator=g).to(torch.bfloat16).to(dev)
    b = torch.randn(k * n, generator=g).to(torch.bfloat16).to(dev)
    bias = torch.randn(n, generator=g).to(torch.bfloat16).to(dev)

    def call():
        c = torch.zeros(m * n, dtype=torch.bfloat16, device=dev)
        gk.gemm_fused(1.0, gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k), 0.0,
                      gk.MatMut.from_row_major(c, m, n), gk.Bias.PerCol(bias), gk.Activation.Relu)
        return c
    *plans_out, single = both(call)
    for o in plans_out[1:]:
        assert torch.equal(bits(o), bits(plans_out[0]))
    with env(**SINGLE):
        assert gk.debug_plan("bf16", "bf16", m, n, 2 * k)[0] == "256x256w8m16"
    ref, got = plans_out[0].float(), single.float()
    floor = 1e-3 * ref.abs().max()
    assert ((got - ref).abs() <= 1e-2 * torch.maximum(ref.abs(), floor)).all()


def test_f32(dev):
    m, k, n = 2048, 2048, 8448
    plans(("f32", "f32", m, n, 4 * k), wide=False)  # f32 inputs never take the wide plan
    g = torch.Generator().manual_seed(8)
    a = torch.rand(m * k, generator=g).to(dev) * 2 - 1
    b = torch.rand(k * n, generator=g).to(dev) * 2 - 1

    def call():
        c = torch.zeros(m * n, dtype=torch.float32, device=dev)
        gk.gemm(1.0, gk.MatRef.from_row_major(a, m, k), gk.MatRef.from_row_major(b, k, n), 0.0,
                gk.MatMut.from_row_major(c, m, n))
        return c
    *plans_out, single = both(call)
    for o in plans_out:
        assert torch.equal(bits(o), bits(single))


@pytest.mark.parametrize("kind", ["i32", "q8"])
def test_ragged_pitched_rest(dev, kind):
    """2000 x 11000 x 4096: by default 8 x 32 tiles of 256 x 352 at a
    344-column pitch (partial last tile row); with that off, the tail split's rest (2000 x 2808) runs
    as 16 x 16 tiles of 128 x 192 at a 176-column pitch (i32), or 16 x 32
    tiles of 128 x 96 at an 88-column pitch, two per CU (requantized), with a
    partial last tile row and column; beta = 1 checks that the overlapping
    columns are stored once."""
    m, k, n = 2000, 4096, 11000
    plans(("i8", kind, m, n, k))
    with env(**SPLIT):
        plan = gk.debug_plan("i8", kind, m, n, k)
    assert plan[2] == ("128x96k128o2" if kind == "q8" else "128x192k128")
    with env(**DEFAULT):
        assert gk.debug_plan("i8", kind, m, n, k, pitches=True)[1] == 344
    a, b = rand_i8(m * k, 9, dev, -127), rand_i8(n * k, 10, dev, -127)
    if kind == "i32":
        g = torch.Generator().manual_seed(11)
        c0 = torch.randint(-1000, 1000, (m * n,), dtype=torch.int32, generator=g).to(dev)

        def call():
            c = c0.clone()
            gk.gemm_i8(1, gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k), 1,
                       gk.MatMut.from_row_major(c, m, n))
            return c
    else:
        g = torch.Generator().manual_seed(12)
        scales = (1e-4 + torch.rand(n, generator=g) * (1e-2 - 1e-4)).to(dev)
        req = gk.Requantize(gk.RequantScale.PerCol(scales), zero_point=5)

        def call():
            c = torch.zeros(m * n, dtype=torch.int8, device=dev)
            gk.gemm_i8_requant(gk.MatRef.from_row_major(a, m, k), gk.MatRef(b, k, n, 1, k), req,
                               gk.MatMut.from_row_major(c, m, n))
            return c
    *plans_out, single = both(call, i8=True)
    for o in plans_out:
        assert torch.equal(o, single)
