"""The prox entry points under HIP graph capture.

The bench replays its launch-bound workloads (C1 and the biased knapsack on
the C1 input) from a captured graph.  Each replay must give what the eager
calls give: the capture records the register kernel, and for the listed
operators the deferred-column kernel whose last workgroup resets the list's
counters for the next replay.  Replays run several times, with the program's
own eager work and synchronisations between them, and every replay is
compared with the eager result.
"""
import numpy as np
import pytest

from tests import inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("op,kw,m", [
    ("knapsack_eq", dict(lo=0.0, hi=1.0, rhs=1.0), 10),
    ("knapsack_le_biased", dict(lo=0.0, hi=1.0, rhs=1.0, rho=1.0), 10),
    ("topk_simplex", dict(k=5, rhs=1.0), 100),
    ("topk_cone", dict(k=5), 100),
])
def test_prox_graph_replays_match_eager(cuda, op, kw, m):
    import torch
    import libsdca_amd as sd
    n = 5000
    dt = torch.float64 if m == 10 else torch.float32
    npdt = np.float64 if m == 10 else np.float32
    xs = [torch.from_numpy(inputs.mixed_signs(n, m, npdt, 300 + i, -2, 2)).to(cuda) for i in range(3)]
    xs[1][::7] = 0.0  # zero-band ties: deferred columns for the cone search
    outs = [torch.empty_like(x) for x in xs]
    eager = []
    for x in xs:
        o = torch.empty_like(x)
        sd.prox(op, x, out=o, **kw)
        eager.append(o)
    torch.cuda.synchronize()
    gs = torch.cuda.Stream()
    with torch.cuda.stream(gs):
        for x, o in zip(xs, outs):  # warm the side stream's workspace before capture
            sd.prox(op, x, out=o, **kw)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=gs):
        for x, o in zip(xs, outs):
            sd.prox(op, x, out=o, **kw)
    torch.cuda.synchronize()
    for rep in range(4):
        for o in outs:
            o.fill_(-7.0)
        g.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), f"{op}: replay {rep}, step {i} differs from the eager call"
        # eager work on the default stream between replays
        tmp = torch.empty_like(xs[0])
        sd.prox(op, xs[0], out=tmp, **kw)
        torch.cuda.synchronize()
        assert torch.equal(tmp, eager[0])


def test_capture_on_a_cold_stream_is_refused(cuda):
    """Scratch cannot grow inside a capture (its wait and allocation are not
    capturable); the call says so instead of invalidating the capture."""
    import torch
    import libsdca_amd as sd
    x = torch.from_numpy(inputs.mixed_signs(4096, 100, np.float32, 310, -2, 2)).to(cuda)
    o = torch.empty_like(x)
    gs = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(sd.SdcaError, match="captured"):
        with torch.cuda.graph(g, stream=gs):
            sd.prox("topk_simplex", x, out=o, k=5, rhs=1.0)
    torch.cuda.synchronize()
    sd.prox("topk_simplex", x, out=o, k=5, rhs=1.0)  # the library still works afterwards
    ref = torch.empty_like(x)
    sd.prox("topk_simplex", x, out=ref, k=5, rhs=1.0)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)


def test_host_threads_sharing_a_stream(cuda):
    """Two host threads that enqueue on one stream, each growing its scratch,
    give what one thread gives: each thread has its own scratch, so a
    growth never frees a buffer the other thread's call is about to use."""
    import threading
    import torch
    import libsdca_amd as sd
    sizes = [1000, 8000, 30000, 120000]
    xs = [torch.from_numpy(inputs.mixed_signs(n, 100, np.float32, 320 + i, -2, 2)).to(cuda)
          for i, n in enumerate(sizes)]
    expect = []
    for x in xs:
        o = torch.empty_like(x)
        sd.prox("topk_cone", x, out=o, k=5)
        expect.append(o)
    torch.cuda.synchronize()
    got = {}
    errors = []

    def worker(t):
        try:
            torch.cuda.set_device(cuda)
            order = sizes if t == 0 else sizes[::-1]
            outs = []
            for n in order:
                i = sizes.index(n)
                o = torch.empty_like(xs[i])
                sd.prox("topk_cone", xs[i], out=o, k=5)
                outs.append((i, o))
            got[t] = outs
        except Exception as e:  # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for t in range(2):
        for i, o in got[t]:
            assert torch.equal(o, expect[i]), f"thread {t}, size {sizes[i]}"
