"""GPU parity of the prefill contract (bf16 activations, exact Q2_0 block scales, bf16 MFMA with f32
accumulation), through the C ABI, against the oracle's or_moe_prefill on the same seeded inputs.

The router runs on the matrix cores (bf16 routers): its logits are within 1e-5 rel_l1 per token of the exact dot,
and the routing (ids, weights) and the dispatch (counts, offsets, perm, slot) of the device's logits are bit-exact
(tests/prefill_check.py); the f32 router's logits are the oracle's bits.  The output is within max rel_l1 1e-3 per
row (metal/src/pack_parity.cpp:2425-2433; the block's gate) of the contract routed from the same logits, the oracle
summing each row in double.  Covers the benchmark's Zipf prefill (config 3), an expert hot enough to split into
several 128-column work items, a shared expert wider than the routed ones, a layer without a shared expert,
a forced MFMA call below the automatic threshold, and the reference model's H=2560 / F=640 shape."""
import os
import sys

import numpy as np
import pytest

import oracle as O
import prefill_check as PC
import stratametal_amd as S

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GUARD = 16
TOL = 1e-3  # max rel_l1 per output row


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


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(torch, t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def hot_bias(E, hot, lift=10.0):
    b = np.zeros(E, np.float32)
    b[hot] = lift
    return b


CASES = [
    # name, geometry, T, seed, add_shared, bias, path
    ("golden small, forced MFMA", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4), 3, 4242, True,
     None, S.PATH_MFMA),
    ("config 3 (prefill 512, Zipf 1.2)", {}, 512, 3, True, "zipf", S.PATH_AUTO),
    ("hot expert split over 3 items", dict(n_embd=256, n_ff=256, n_ff_shared=128, n_expert=16, top_k=2), 300, 11,
     True, ("hot", 5), S.PATH_AUTO),
    ("shared wider than routed", dict(n_embd=512, n_ff=128, n_ff_shared=256, n_expert=32, top_k=4), 130, 12, True,
     None, S.PATH_AUTO),
    ("no shared expert", dict(n_embd=512, n_ff=256, sh_type=-1, n_expert=64, top_k=6), 200, 13, True, None,
     S.PATH_AUTO),
    ("shared not added", dict(n_embd=512, n_ff=256, n_expert=64, top_k=6), 129, 14, False, None, S.PATH_AUTO),
    ("reference model shape H=2560 F=640", dict(n_embd=2560, n_ff=640, n_ff_shared=640, n_expert=64, top_k=8), 160,
     15, True, None, S.PATH_AUTO),
    ("7 experts top-3, 9 tokens forced", dict(n_embd=256, n_ff=256, n_ff_shared=128, n_expert=7, top_k=3), 9, 8, True,
     None, S.PATH_MFMA),
    # 20000 pairs over 20 dispatch chunks, a hot expert whose pairs span every chunk and many work items
    ("many pairs, hot expert", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=64, top_k=8), 2500, 16, True,
     ("hot", 9), S.PATH_AUTO),
    # 1024 experts, every one touched, almost all with a remainder item of 2..64 columns: the item-class counts
    # reach 1024 (the packed scan fields must hold it)
    ("1024 experts all touched", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=1024, top_k=8), 2048, 18,
     True, None, S.PATH_AUTO),
    # 8000 pairs: eight dispatch chunks over 1024 experts, the most that the dispatch scan counts in its own LDS
    ("8 dispatch chunks over 1024 experts", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=1024, top_k=8),
     1000, 29, True, None, S.PATH_AUTO),
    # the f32 router (router_dtype 1) on the prefill path: the row-per-wave router over f32 token tiles
    ("f32 router, prefill 512 Zipf 1.2", dict(router_dtype=1), 512, 19, True, "zipf", S.PATH_AUTO),
    ("f32 router, 200 tokens", dict(router_dtype=1, n_embd=512, n_ff=256, n_expert=64, top_k=6), 200, 20, True, None,
     S.PATH_AUTO),
    # about three pairs per expert at the configs' geometry: nearly every routed item (and the shared remainder
    # chunk of 32) is a thin work item
    ("config geometry, 160 tokens (thin items)", {}, 160, 21, True, None, S.PATH_AUTO),
    ("600 experts top-10, 300 tokens", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=600, top_k=10), 300, 23,
     True, None, S.PATH_AUTO),
    # long down K loops (16 units) and 16 gate/up row blocks; the widest rows of the router tile (H 4096)
    ("n_ff 2048, 200 tokens", dict(n_embd=512, n_ff=2048, n_ff_shared=2048, n_expert=32, top_k=4), 200, 24, True,
     None, S.PATH_AUTO),
    ("H=4096, 140 tokens", dict(n_embd=4096, n_ff=256, n_ff_shared=256, n_expert=16, top_k=4), 140, 25, True, None,
     S.PATH_AUTO),
    ("H=1024 F=512, 136 tokens (thin items, a shared remainder of 8)",
     dict(n_embd=1024, n_ff=512, n_ff_shared=512, n_expert=128, top_k=4), 136, 22, True, None, S.PATH_AUTO),
    # H 1536: 12 units (three four-unit thin stages); n_ff 384: three gate/up row blocks, down rows of three units
    ("H=1536 F=384, 150 tokens", dict(n_embd=1536, n_ff=384, n_ff_shared=384, n_expert=64, top_k=4), 150, 26, True,
     None, S.PATH_AUTO),
    # H 384: one down work-group takes both row blocks, the second only half there (its rows past H read as zeros)
    ("H=384, 140 tokens (a half down row block)", dict(n_embd=384, n_ff=256, n_ff_shared=256, n_expert=32, top_k=4),
     140, 27, True, None, S.PATH_AUTO),
    # H 640: three down row blocks, a pair and a half block alone
    ("H=640, 140 tokens", dict(n_embd=640, n_ff=256, n_ff_shared=256, n_expert=32, top_k=4), 140, 28, True, None,
     S.PATH_AUTO),
]

_LAYERS = {}


def layer(torch, g, seed, bias):
    key = (tuple(vars(g).values()), seed, None if bias is None else bias.tobytes())
    if key not in _LAYERS:
        _LAYERS.clear()
        w_host = O.make_weights(g, seed, zipf_bias=bias)
        w_dev = S.synth_layer(S.Geom(**vars(g)), seed, logit_bias=None if bias is None else dev(torch, bias))
        _LAYERS[key] = (w_host, w_dev)
    return _LAYERS[key]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_forward_prefill_parity(torch, case):
    name, gkw, T, seed, add_shared, bias, path = CASES[case]
    say(f"case: prefill {name} T={T}")
    g = O.Geom(**gkw)
    if bias == "zipf":
        bias = S.zipf_bias(g.n_expert, 1.2, seed, n_tokens=T, top_k=g.top_k, n_embd=g.n_embd)
    elif isinstance(bias, tuple):
        bias = hot_bias(g.n_expert, bias[1])
    w_host, w_dev = layer(torch, g, seed, bias)
    x = O.gen_normal(seed, 100, T * g.n_embd).reshape(T, g.n_embd)
    ml = S.MoELayer(S.Geom(**vars(g)), w_dev, max_tokens=T)
    yg = torch.full((T * g.n_embd + GUARD,), 7.0, dtype=torch.float32, device="cuda")
    yv = yg[:T * g.n_embd].view(T, g.n_embd)
    _, tr = ml.forward(dev(torch, x), y=yv, add_shared=add_shared, trace=True, path=path)
    got = host(torch, yg)
    assert (got[T * g.n_embd:] == 7.0).all(), "guard words past y were written"
    y = got[:T * g.n_embd].reshape(T, g.n_embd)
    htr = {k: host(torch, v) for k, v in tr.items()}
    # the router stage by stage (its logits on the matrix cores, the routing of those logits exact), then the block
    # against the prefill contract routed from the same logits
    worst = PC.router_stagewise(g, w_host, x, htr)
    want = PC.prefill_want(g, w_host, x, htr, add_shared=add_shared, n_threads=16)
    if g.router_dtype == 1:  # the f32 router runs row per wave on every path: the oracle's bits
        _, wtr = O.moe_prefill(g, w_host, x, add_shared=add_shared, trace=True, n_threads=16)
        assert np.array_equal(bits(htr["logits"]), bits(wtr["logits"]))
    err = O.rel_l1_rows(y, want)
    counts = host(torch, tr["counts"])
    say(f"  max rel_l1 {err.max():.3e} (mean {err.mean():.3e}); logits {worst:.2e} from the exact dot; "
        f"hottest expert {counts.max()} pairs")
    assert err.max() <= TOL
    if name.startswith("hot"):
        assert counts.max() > 2 * S.MFMA_CHUNK, "the hot expert does not span three work items"
    if name.startswith("1024"):
        assert (counts > 0).all() and counts.max() <= S.MFMA_CHUNK // 2, "not every expert holds a short remainder"
    if name.startswith("golden"):
        f = np.load(os.path.join(GOLD, "layer_prefill.npz"))
        assert np.array_equal(bits(x), bits(f["x"]))
        assert O.rel_l1_rows(y, f["y"]).max() <= TOL
    # determinism: a repeat is bitwise identical
    y2 = ml.forward(dev(torch, x), add_shared=add_shared, path=path)
    assert np.array_equal(bits(host(torch, y2)), bits(y))


def test_trace_stages_and_fp16_overflow_mask(torch):
    """The prefill path's trace: parts and shared within the contract's 1e-3 per row of the oracle's; the overflow
    mask 0 for ordinary inputs, bit 0 for a token whose activations reach the fp16 limit (65520), bit 1 for one
    whose h does, the other tokens' outputs unaffected; the decode path reports 0 on the same inputs."""
    say("case: prefill trace stages and fp16 overflow mask")
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4)
    w_host, w_dev = layer(torch, g, 31, None)
    T = 160
    ml = S.MoELayer(S.Geom(**vars(g)), w_dev, max_tokens=T)
    x = O.gen_normal(31, 100, T * g.n_embd).reshape(T, g.n_embd)
    y, tr = ml.forward(dev(torch, x), trace=True, stages=True)
    htr = {k: host(torch, v) for k, v in tr.items()}
    PC.router_stagewise(g, w_host, x, htr)
    want, wtr = PC.prefill_want(g, w_host, x, htr, trace=True, n_threads=16)
    assert host(torch, tr["overflow"])[0] == 0
    assert O.rel_l1_rows(host(torch, y), want).max() <= TOL
    assert O.rel_l1_rows(host(torch, tr["parts"]), wtr["parts"]).max() <= TOL
    assert O.rel_l1_rows(host(torch, tr["shared"]), wtr["shared"]).max() <= TOL
    for bad, scale, bit in ((7, 1e5, 1), (9, 1e3, 2)):
        xb = x.copy()
        xb[bad] *= scale
        yb, trb = ml.forward(dev(torch, xb), trace=True, stages=True)
        mask = int(host(torch, trb["overflow"])[0])
        assert mask == bit, (scale, mask)
        yw = PC.prefill_want(g, w_host, xb, {k: host(torch, v) for k, v in trb.items()}, n_threads=16)
        assert np.isfinite(yw).all(), "the oracle holds the contract beyond the fp16 limit"
        keep = np.arange(T) != bad
        assert O.rel_l1_rows(host(torch, yb)[keep], yw[keep]).max() <= TOL
        # the decode path has no such limit: it reports 0 on the same tokens
        _, trd = ml.forward(dev(torch, xb[bad - 2:bad + 2]), trace=True, stages=True)
        assert host(torch, trd["overflow"])[0] == 0


def test_auto_path_switches_at_128_tokens(torch):
    """SMOE_PATH_AUTO runs the decode contract below 128 tokens and the prefill contract from 128 on."""
    say("case: automatic path threshold")
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4)
    w_host, w_dev = layer(torch, g, 21, None)
    x = O.gen_normal(21, 100, 128 * g.n_embd).reshape(128, g.n_embd)
    ml = S.MoELayer(S.Geom(**vars(g)), w_dev, max_tokens=128)
    y127 = host(torch, ml.forward(dev(torch, x[:127])))
    assert np.array_equal(bits(y127), bits(O.moe_decode_dev(g, w_host, x[:127], n_threads=16)))
    y128, tr = ml.forward(dev(torch, x), trace=True)
    htr = {k: host(torch, v) for k, v in tr.items()}
    PC.router_stagewise(g, w_host, x, htr)
    y128 = host(torch, y128)
    assert O.rel_l1_rows(y128, PC.prefill_want(g, w_host, x, htr, n_threads=16)).max() <= TOL
    # and the two contracts differ (q8_1 vs bf16 activations), so the switch is observable
    assert not np.array_equal(bits(y128[:127]), bits(y127))
