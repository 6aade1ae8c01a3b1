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
