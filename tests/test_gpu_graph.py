"""GPU test of the block under HIP graph capture: a chain of layer calls that covers every launch sequence (one token:
router + the fused small-batch launch; three tokens; sixteen tokens: router, top-k, dispatch, gate/up, down,
combine; 160 tokens: the MFMA contract) is captured once and replayed three times, with the program's own eager
calls and synchronisations between the replays, and every replay's outputs equal the eager calls' bit for bit.
The calls share one workspace, so a replay also shows that no launch depends on what an earlier one left there
(the fused launch's exchange words are cleared inside the call, by a kernel, not by a memset node)."""
import sys

import numpy as np
import pytest

import stratametal_amd as S

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as T
    if not T.cuda.is_available():
        pytest.skip("no GPU")
    S.lib()
    return T


def test_graph_replays_equal_eager_calls(torch):
    say("case: graph capture of 1/3/16/160-token calls, 3 replays")
    g = S.Geom()
    H = g.n_embd
    sizes = (1, 3, 16, 160, 1)
    layers = [S.MoELayer(g, S.synth_layer(g, 7100 + i), max_tokens=max(sizes)) for i in range(2)]
    xs = [S.synth_normal(7200 + i, 100, T * H).view(T, H) for i, T in enumerate(sizes)]
    ys = [torch.empty_like(x) for x in xs]

    def chain():
        for i, x in enumerate(xs):
            layers[i % 2].forward(x, ys[i])

    chain()
    torch.cuda.synchronize()
    want = [y.clone() for y in ys]
    graph = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(graph, stream=st):
            chain()
    torch.cuda.synchronize()
    for rep in range(3):
        for y in ys:
            y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for i, (y, w) in enumerate(zip(ys, want)):
            assert torch.equal(y.view(torch.int32), w.view(torch.int32)), (rep, sizes[i])
        # the program's own eager work between replays, on the same workspaces
        layers[0].forward(xs[2][:5])
        torch.cuda.synchronize()
    assert all(bool(torch.isfinite(w).all()) for w in want)
