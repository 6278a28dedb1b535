"""Every route of the library captured into one HIP graph (stream-ordered
calls, a workspace sized beforehand) and replayed several times, with eager
work on the same buffers between the replays: each replay must reproduce the
eager results bit for bit.  Routes: the 256 x 256 tile kernel, a packed
operand, split K with its reduction, the one-round 256 x 352 plan and the
tail split with its pitched rest (requantized), the short-contraction
streaming kernel, the wavefront GEMV, the skinny kernel with strided
activations, the small f32 kernel and a fused bf16 epilogue.  (No route records a memset: every scratch value is written
before it is read.)"""
import os

import pytest
import torch

import gemmkit_amd as gk

pytestmark = pytest.mark.gpu


def _i8(n, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-127, 128, (n,), dtype=torch.int8, generator=g).to(dev)


def _f(n, seed, dev, dt=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, generator=g).to(dt).to(dev)


def build_calls(dev, ws):
    """(name, output tensor, call) for each route (shapes bound at creation)."""
    calls = []
    # 256 x 256 tiles, i32 out, alpha/beta
    m = k = n = 1024
    a1, b1 = _i8(m * k, 1, dev), _i8(k * n, 2, dev)
    c1 = torch.zeros(m * n, dtype=torch.int32, device=dev)
    calls.append(("i8 tiles", c1, lambda m=m, k=k, n=n: gk.gemm_i8(
        2, gk.MatRef.from_row_major(a1, m, k), gk.MatRef(b1, k, n, 1, k), 1,
        gk.MatMut.from_row_major(c1, m, n), ws=ws)))
    # f32 with a row-major B (packed into the workspace), tile route
    m = k = n = 768
    a2, b2 = _f(m * k, 3, dev), _f(k * n, 4, dev)
    c2 = torch.zeros(m * n, device=dev)
    calls.append(("f32 packed B", c2, lambda m=m, k=k, n=n: gk.gemm(
        1.0, gk.MatRef.from_row_major(a2, m, k), gk.MatRef.from_row_major(b2, k, n), 0.0,
        gk.MatMut.from_row_major(c2, m, n), ws=ws)))
    # i8 split K (few 64 x 64 tiles, long K) with its reduction
    m, k, n = 128, 8192, 192
    a3, b3 = _i8(m * k, 5, dev), _i8(k * n, 6, dev)
    c3 = torch.zeros(m * n, dtype=torch.int32, device=dev)
    calls.append(("i8 split K", c3, lambda m=m, k=k, n=n: gk.gemm_i8(
        1, gk.MatRef.from_row_major(a3, m, k), gk.MatRef(b3, k, n, 1, k), 0,
        gk.MatMut.from_row_major(c3, m, n), ws=ws)))
    # requantized 2000 x 11000 x 4096: one round of 256 x 352 tiles at a
    # column pitch, and (GEMMKIT_HIP_WIDE=0 while the call is made) the tail
    # split with its pitched rest
    m, k, n = 2000, 4096, 11000
    a4, b4 = _i8(m * k, 7, dev), _i8(n * k, 8, dev)
    g = torch.Generator().manual_seed(9)
    sc = (1e-4 + torch.rand(n, generator=g) * 1e-2).to(dev)
    req = gk.Requantize(gk.RequantScale.PerCol(sc), zero_point=3, relu=True)
    c4 = torch.zeros(m * n, dtype=torch.int8, device=dev)
    calls.append(("requant wide round", c4, lambda m=m, k=k, n=n: gk.gemm_i8_requant(
        gk.MatRef.from_row_major(a4, m, k), gk.MatRef(b4, k, n, 1, k), req,
        gk.MatMut.from_row_major(c4, m, n), ws=ws)))
    c4s = torch.zeros(m * n, dtype=torch.int8, device=dev)

    def split_call(m=m, k=k, n=n):
        os.environ["GEMMKIT_HIP_WIDE"] = "0"
        try:
            gk.gemm_i8_requant(gk.MatRef.from_row_major(a4, m, k), gk.MatRef(b4, k, n, 1, k), req,
                               gk.MatMut.from_row_major(c4s, m, n), ws=ws)
        finally:
            del os.environ["GEMMKIT_HIP_WIDE"]
    calls.append(("requant tail split", c4s, split_call))
    # batched short contraction (streaming kernel)
    bt, s, d = 8, 256, 64
    q, kk = _f(bt * s * d, 10, dev, torch.bfloat16), _f(bt * s * d, 11, dev, torch.bfloat16)
    c5 = torch.zeros(bt * s * s, device=dev)
    calls.append(("bf16 batched short K", c5, lambda: gk.gemm_batched_bf16_f32out(
        bt, 0.125, gk.MatRef.from_row_major(q, s, d), s * d, gk.MatRef(kk, d, s, 1, d), s * d,
        0.0, gk.MatMut.from_row_major(c5, s, s), s * s, ws=ws)))
    # GEMV (one activation row) and skinny (8 column-major activation rows)
    nw, k = 4096, 4096
    w = _i8(nw * k, 12, dev)
    x1 = _i8(k, 13, dev)
    c6 = torch.zeros(nw, dtype=torch.int32, device=dev)
    calls.append(("i8 GEMV", c6, lambda k=k: gk.gemm_i8(
        1, gk.MatRef.from_row_major(x1, 1, k), gk.MatRef(w, k, nw, 1, k), 0,
        gk.MatMut.from_row_major(c6, 1, nw), ws=ws)))
    x8 = _i8(8 * k, 14, dev)
    c7 = torch.zeros(8 * nw, dtype=torch.int32, device=dev)
    calls.append(("i8 skinny", c7, lambda k=k: gk.gemm_i8(
        1, gk.MatRef.from_col_major(x8, 8, k), gk.MatRef(w, k, nw, 1, k), 0,
        gk.MatMut.from_row_major(c7, 8, nw), ws=ws)))
    # small f32, all row-major
    m = k = n = 512
    a8, b8 = _f(m * k, 15, dev), _f(k * n, 16, dev)
    c8 = torch.zeros(m * n, device=dev)
    calls.append(("f32 small", c8, lambda m=m, k=k, n=n: gk.gemm(
        1.0, gk.MatRef.from_row_major(a8, m, k), gk.MatRef.from_row_major(b8, k, n), 0.0,
        gk.MatMut.from_row_major(c8, m, n), ws=ws)))
    # fused bf16 (bias per column, LeakyReLU)
    m, k, n = 600, 512, 700
    a9, b9 = _f(m * k, 17, dev, torch.bfloat16), _f(k * n, 18, dev, torch.bfloat16)
    bias = _f(n, 19, dev, torch.bfloat16)
    c9 = torch.zeros(m * n, dtype=torch.bfloat16, device=dev)
    calls.append(("bf16 fused", c9, lambda m=m, k=k, n=n: gk.gemm_fused(
        1.0, gk.MatRef.from_row_major(a9, m, k), gk.MatRef(b9, k, n, 1, k), 0.0,
        gk.MatMut.from_row_major(c9, m, n), gk.Bias.PerCol(bias), gk.Activation.LeakyRelu(0.1),
        ws=ws)))
    return calls


def test_captured_requant_needs_checked_scales(dev):
    """The checked requantizing entry copies per-channel scales back to check
    them; under capture it accepts only scales an uncaptured call on this
    thread has checked, and otherwise fails with a clear error (the capture
    is then invalid, as for any failed capture)."""
    m, k, n = 64, 128, 96
    a, b = _i8(m * k, 30, dev), _i8(k * n, 31, dev)
    sc = torch.full((n,), 0.01, device=dev)
    req = gk.Requantize(gk.RequantScale.PerCol(sc))
    c = torch.zeros(m * n, dtype=torch.int8, device=dev)
    gk.set_synchronous(False)
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        err = None
        graph = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.stream(side):
                with torch.cuda.graph(graph, stream=side):
                    try:
                        gk.gemm_i8_requant(gk.MatRef.from_row_major(a, m, k),
                                           gk.MatRef(b, k, n, 1, k), req,
                                           gk.MatMut.from_row_major(c, m, n))
                    except gk.GemmkitError as e:
                        err = str(e)
        except Exception:
            pass
        assert err is not None and "graph capture" in err, err
    finally:
        gk.set_synchronous(True)
    torch.cuda.synchronize()


def test_every_route_replays_bit_exact(dev):
    ws = gk.Workspace.with_capacity(256 << 20)
    calls = build_calls(dev, ws)
    # eager references (synchronous calls)
    want = {}
    for name, out, fn in calls:
        out.zero_()
        fn()
        want[name] = out.clone()
    gk.set_synchronous(False)
    try:
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for _, _, fn in calls:
                    fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for rep in range(3):
            # eager work on the same buffers between replays: clear the
            # outputs (the i32 tiles call accumulates with beta = 1, so it is
            # reset to its starting zeros) and run one route eagerly
            for _, out, _ in calls:
                out.zero_()
            dict((nm, fn) for nm, _, fn in calls)["i8 GEMV"]()
            torch.cuda.synchronize()
            for _, out, _ in calls:
                out.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for name, out, _ in calls:
                assert torch.equal(out, want[name]), (rep, name)
    finally:
        gk.set_synchronous(True)
