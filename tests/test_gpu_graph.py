"""GPU test of the block under HIP graph capture: a chain of layer calls that covers every launch sequence (one token:
router + the fused small-batch launch; three tokens; sixteen tokens: router, top-k, dispatch, gate/up, down,
combine; 160 tokens: the MFMA contract) is captured once and replayed three times, with the program's own eager
calls and synchronisations between the replays, and every replay's outputs equal the eager calls' bit for bit.
The calls share one workspace, so a replay also shows that no launch depends on what an earlier one left there
(the fused launch's exchange words are cleared inside the call, by a kernel, not by a memset node).  Also: the
other call sequences under capture, and calls on two streams at once."""
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


def test_graph_replays_other_paths(torch):
    """The other call sequences under capture: IQ2_S layers (1, 3 and 64 tokens), the f32 router (1 and 16 tokens),
    the stack junction fused into the call (1 and 130 tokens) and the hyper-connection layer call (1 token), captured
    once and replayed three times with eager work between; every replay equals the eager calls bit for bit."""
    import oracle as O
    say("case: graph capture of IQ2_S, f32 router, fused junction and hyper-connection calls, 3 replays")
    g, gi, gf = S.Geom(), S.Geom(w_type=22, sh_type=22), S.Geom(router_dtype=1)
    H = g.n_embd
    li = S.MoELayer(gi, S.synth_layer(gi, 7300), max_tokens=64)
    lf = S.MoELayer(gf, S.synth_layer(gf, 7301), max_tokens=16)
    wq = S.synth_layer(g, 7302)
    lr = S.MoELayer(g, wq, max_tokens=130)
    hw = O.make_hc(H, 4, 320, 7303)
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    hcx = S.HyperConnection(H, hw.hc, hw.hc_lr, to(hw.norm), to(hw.down.view(np.int16)), to(hw.up.view(np.int16)),
                            to(hw.inject.view(np.int16)), eps=hw.eps)
    lh = S.FfnLayer(g, wq, hcx, max_tokens=1)
    x = {T: S.synth_normal(7400 + T, 100, T * H).view(T, H) for T in (1, 3, 16, 64, 130)}
    r = {T: S.synth_normal(7500 + T, 100, T * H).view(T, H) for T in (1, 130)}
    R = S.synth_normal(7600, 100, 4 * H).view(1, 4, H)
    outs = {}

    def chain():
        for T in (1, 3, 64):
            outs[("iq2", T)] = li.forward(x[T])
        for T in (1, 16):
            outs[("f32", T)] = lf.forward(x[T])
        for T in (1, 130):
            xj = outs.setdefault(("xj", T), torch.empty_like(x[T]))
            outs[("res", T)] = lr.forward_residual(x[T], r[T], xj)
        outs[("hc", 1)] = lh.run(R)

    chain()
    torch.cuda.synchronize()
    want = {k: v.clone() for k, v in outs.items()}
    graph = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(graph, stream=st):
            chain()
    torch.cuda.synchronize()
    for rep in range(3):
        for v in outs.values():
            v.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for k, v in outs.items():
            assert torch.equal(v.view(torch.int32), want[k].view(torch.int32)), (rep, k)
        li.forward(x[3])  # the program's own eager work between replays, on the same workspaces
        lr.forward(x[1])
        torch.cuda.synchronize()
    assert all(bool(torch.isfinite(w).all()) for w in want.values())


def test_concurrent_calls_on_two_streams(torch):
    """Two layers with their own workspaces called on two streams (default priority) with no synchronisation
    between them, at 1 token (the fused launch, whose down work-groups wait for the h words of their own launch),
    16 and 130 tokens: every output equals the same calls run one after another, bit for bit."""
    say("case: concurrent calls on two streams, 1/16/130 tokens")
    g = S.Geom()
    H = g.n_embd
    layers = [S.MoELayer(g, S.synth_layer(g, 7700 + i), max_tokens=130) for i in range(2)]
    for T in (1, 16, 130):
        xs = [S.synth_normal(7800 + 10 * T + i, 100, T * H).view(T, H) for i in range(2)]
        want = [layers[i].forward(xs[i]) for i in range(2)]
        torch.cuda.synchronize()
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        got = [None, None]
        for rep in range(4):  # the two streams' launches interleave
            for i in range(2):
                with torch.cuda.stream(streams[i]):
                    got[i] = layers[i].forward(xs[i])
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(got[i].view(torch.int32), want[i].view(torch.int32)), (T, i)
