"""The workspace across streams.  The reference's Workspace has one user at a
time (`&mut Workspace`, src/workspace.rs:53-60); here stream-ordered calls on
different streams may share one arena (the thread's own, or a caller's), so a
call on another stream than the arena's last user first waits for that user's
work.  Each product below packs its row-major B into the arena; the calls
alternate between two streams without any host synchronization, so without
that ordering the second call's pack would overwrite the first call's packed
B while the first call's kernel still reads it.  Every result is checked
against the same product computed synchronously (i8 results are exact)."""
import pytest
import torch

import gemmkit_amd as gk

pytestmark = pytest.mark.gpu


def _i8(n, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-127, 128, (n,), dtype=torch.int8, generator=g).to(dev)


@pytest.mark.parametrize("own_ws", [False, True])
def test_async_packs_on_two_streams_stay_ordered(own_ws):
    dev = torch.device("cuda:0")
    m, k, n = 2048, 4096, 2048
    ws = gk.Workspace() if own_ws else None
    sets = []
    for i in range(4):
        a = _i8(m * k, 10 + 2 * i, dev)
        b = _i8(k * n, 11 + 2 * i, dev)  # row-major k x n: its B^T is packed
        sets.append((a, b))

    def call(a, b, c):
        gk.gemm_i8(1, gk.MatRef.from_row_major(a, m, k), gk.MatRef.from_row_major(b, k, n), 0,
                   gk.MatMut.from_row_major(c, m, n), ws=ws)

    want = []
    for a, b in sets:
        c = torch.empty(m * n, dtype=torch.int32, device=dev)
        call(a, b, c)  # synchronous (the default)
        want.append(c)
    torch.cuda.synchronize()

    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    gk.set_synchronous(False)
    try:
        for rnd in range(3):
            outs = [torch.full((m * n,), -1, dtype=torch.int32, device=dev) for _ in sets]
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(sets):
                with torch.cuda.stream(streams[(i + rnd) % 2]):
                    call(a, b, outs[i])
            torch.cuda.synchronize()
            for i, o in enumerate(outs):
                assert torch.equal(o, want[i]), f"round {rnd}, product {i} differs"
    finally:
        gk.set_synchronous(True)
        torch.cuda.synchronize()
    del ws
