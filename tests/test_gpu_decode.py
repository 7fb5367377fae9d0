"""GPU parity of the decode contract, through the C ABI (libsmoe.so), against the oracle on the same seeded
inputs.  Bitwise against the oracle's device-order restatement (or_*_dev); within the reference's own bounds
against its reference-order chain (1e-5 per stage, 1e-3 per output row, metal/src/pack_parity.cpp:8764-8770);
ids and dispatch permutations bit-exact.  Guard words past every output stay put (7.0), zero counts leave
outputs untouched, refused calls launch nothing, repeats are bitwise identical."""
import os
import sys

import numpy as np
import pytest

import oracle as O
import stagewise as SW
import stratametal_amd as S

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GUARD = 16


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


def guarded(torch, n, dtype):
    t = torch.full((n + GUARD,), 7, dtype=dtype, device="cuda")
    return t


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def stage_pass(torch, ml, x, add_shared):
    """A traced pass with the expert stages: (host copies of the trace, host y)."""
    y, tr = ml.forward(dev(torch, x), add_shared=add_shared, trace=True, stages=True)
    return {k: host(torch, v) for k, v in tr.items()}, host(torch, y)


# ------------------------------------------------------------------------------------------------ generators

def test_synth_matches_oracle_bitwise(torch):
    say("case: synth generators")
    for t, n in ((42, 64 * 3000), (22, 256 * 300)):
        buf = torch.empty(n // (64 if t == 42 else 256) * (18 if t == 42 else 82), dtype=torch.uint8, device="cuda")
        S._check(S.lib().smoe_synth_blocks(t, 9, 3, n, 0.02, buf.data_ptr(), S._stream()))
        assert np.array_equal(host(torch, buf), O.gen_blocks(t, 9, 3, n, 0.02)), t
    b = torch.empty(50000, dtype=torch.int16, device="cuda")
    S._check(S.lib().smoe_synth_bf16(5, 4, 50000, 0.02, b.data_ptr(), S._stream()))
    assert np.array_equal(host(torch, b).view(np.uint16), O.gen_bf16(5, 4, 50000, 0.02))
    x = S.synth_normal(11, 100, 100000)
    assert np.array_equal(bits(host(torch, x)), bits(O.gen_normal(11, 100, 100000)))


# ------------------------------------------------------------------------------------------------ stages

def test_quantize_q8_1_bitwise(torch):
    say("case: quantize_q8_1")
    x = O.gen_normal(1, 1, 32 * 1000)
    x[3] = 1e10
    x[40] = -8e6
    x[64:96] = 0.0
    y = S.quantize_q8_1(dev(torch, x))
    assert np.array_equal(host(torch, y), O.quant_q8_1(x))


def test_f32_to_bf16_bitwise(torch):
    say("case: f32_to_bf16")
    rng = np.random.default_rng(3)
    x = rng.integers(0, 2 ** 32, 32 * 4096, dtype=np.uint64).astype(np.uint32).view(np.float32)
    y = S.f32_to_bf16(dev(torch, x))
    assert np.array_equal(host(torch, y).view(np.uint16), O.bf16_from_f32(x))


@pytest.mark.parametrize("H,E,T", [(2048, 512, 1), (2048, 512, 5), (256, 33, 17), (2560, 64, 2)])
def test_bf16_gemv_bitwise(torch, H, E, T):
    say(f"case: bf16_gemv H={H} E={E} T={T}")
    xb = O.gen_bf16(2, 1, T * H, 1.0)
    W = O.gen_bf16(2, 2, E * H, 0.02)
    y = S.bf16_gemv(dev(torch, xb.view(np.int16)), dev(torch, W.view(np.int16)), H, E)
    got = host(torch, y)
    for t in range(T):
        want = O.bf16_gemv_dev(xb[t * H:(t + 1) * H], W, H, E)
        assert np.array_equal(bits(got[t]), bits(want))
        assert O.rel_l1_rows(got[t][None], O.bf16_gemv_double(xb[t * H:(t + 1) * H], W, H, E)[None])[0] <= 1e-5


def _router_cases():
    T, E = 64, 512
    a = O.gen_normal(2024, 1, T * E).reshape(T, E)
    b = np.full((T, E), 0.5, np.float32)
    c = np.minimum(O.gen_normal(2024, 2, T * E).reshape(T, E), 1.9)
    c[:, :12] = 2.0
    d = np.zeros((T, E), np.float32)
    d[np.arange(T), np.arange(T) % E] = 20.0
    return [("random normal", a, 10), ("all equal", b, 10), ("12-way tie", c, 10), ("dominant", d, 10),
            ("7 experts top-3", O.gen_normal(7, 1, 28).reshape(4, 7), 3),
            ("1024 experts", O.gen_normal(7, 2, 4096).reshape(4, 1024), 10),
            ("k = 64", O.gen_normal(7, 3, 128).reshape(2, 64), 64)]


@pytest.mark.parametrize("case", range(7))
def test_router_topk(torch, case):
    name, logits, k = _router_cases()[case]
    say(f"case: router_topk {name}")
    T, E = logits.shape
    ids_t = guarded(torch, T * k, torch.int32)
    w_t = guarded(torch, T * k, torch.float32)
    logits_t = dev(torch, logits)
    S._check(S.lib().smoe_router_topk(logits_t.data_ptr(), T, E, k, ids_t.data_ptr(), w_t.data_ptr(), S._stream()))
    ids, w = host(torch, ids_t), host(torch, w_t)
    assert (ids[T * k:] == 7).all() and (w[T * k:] == 7.0).all()
    ids, w = ids[:T * k].reshape(T, k), w[:T * k].reshape(T, k)
    ids_d, w_d = O.route_dev(logits, k)
    ids_r, w_r = O.route_ref(logits, k)
    assert np.array_equal(ids, ids_d) and np.array_equal(ids, ids_r)
    assert np.array_equal(bits(w), bits(w_d))
    assert np.max(np.abs(w - w_r) / np.abs(w_r)) <= 1e-5
    assert np.max(np.abs(w.sum(axis=1) - 1.0)) <= 1e-5


def test_router_zero_tokens_leaves_buffers(torch):
    say("case: router zero tokens")
    ids_t = guarded(torch, 0, torch.int32)
    S._check(S.lib().smoe_router_topk(ids_t.data_ptr(), 0, 512, 10, ids_t.data_ptr(), ids_t.data_ptr(), S._stream()))
    assert (host(torch, ids_t) == 7).all()


@pytest.mark.parametrize("n_in,n_out,n_col", [(128, 1, 1), (2048, 512, 3), (512, 2048, 1), (2560, 64, 2),
                                              (640, 100, 5), (4096, 8, 9)])
def test_mmvq_q2_0_bitwise(torch, n_in, n_out, n_col):
    say(f"case: mmvq Q2_0 {n_in}x{n_out} cols={n_col}")
    w = O.gen_q2_0(20261014, n_in + n_out, n_out * n_in // 64)
    x = O.gen_normal(20261014, n_col, n_col * n_in)
    xq = O.quant_q8_1(x)
    y = S.mmvq(42, dev(torch, w), dev(torch, xq), n_in, n_out, n_col)
    got = host(torch, y)
    for c in range(n_col):
        xc = xq[c * n_in // 32 * 36:(c + 1) * n_in // 32 * 36]
        assert np.array_equal(bits(got[c]), bits(O.q2_0_gemv_dev(w, xc, n_in, n_out)))
        assert O.rel_l1_rows(got[c][None], O.q2_0_gemv_ref(w, xc, n_in, n_out)[None])[0] <= 1e-5


def test_mmvq_byte_offset_reads_the_up_rows(torch):
    say("case: mmvq byte offset")
    n_in, n_out = 256, 64
    blob = O.gen_q2_0(3, 3, 2 * n_out * n_in // 64)
    xq = O.quant_q8_1(O.gen_normal(3, 4, n_in))
    off = n_out * n_in // 64 * 18
    y = S.mmvq(42, dev(torch, blob), dev(torch, xq), n_in, n_out, 1, byte_off=off)
    assert np.array_equal(bits(host(torch, y)[0]), bits(O.q2_0_gemv_dev(blob[off:], xq, n_in, n_out)))


def test_swiglu_q8_bitwise(torch):
    say("case: swiglu_q8")
    g = O.gen_normal(4, 1, 32 * 512) * 3
    u = O.gen_normal(4, 2, 32 * 512)
    g[:32] = 0
    y = S.swiglu_q8(dev(torch, g), dev(torch, u))
    assert np.array_equal(host(torch, y), O.swiglu_q8(g, u))


@pytest.mark.parametrize("n,k,shared", [(256, 10, True), (2560, 10, True), (2048, 10, False), (64, 64, True)])
def test_combine(torch, n, k, shared):
    say(f"case: combine n={n} k={k} shared={shared}")
    parts = O.gen_normal(31337, n, k * n).reshape(k, n)
    w = np.abs(O.gen_normal(31337, 2, k)) + 0.05
    w = (w / w.sum()).astype(np.float32)
    sh = 3.0 * O.gen_normal(31337, 3, n) if shared else None
    y = guarded(torch, n, torch.float32)
    parts_t, w_t = dev(torch, parts), dev(torch, w)      # held: a dropped temporary's block is reused at once
    sh_t = None if sh is None else dev(torch, sh)
    S._check(S.lib().smoe_combine(parts_t.data_ptr(), w_t.data_ptr(), None if sh_t is None else sh_t.data_ptr(),
                                  y.data_ptr(), n, k, S._stream()))
    got = host(torch, y)
    assert (got[n:] == 7.0).all()
    assert np.array_equal(bits(got[:n]), bits(O.combine_dev(parts, w, sh)))
    assert O.rel_l1_rows(got[:n][None], O.combine_double(parts, w, sh)[None])[0] <= 1e-6


@pytest.mark.parametrize("T,k,E,zipf", [(1, 10, 512, False), (16, 10, 512, False), (97, 10, 64, False),
                                        (512, 10, 512, True), (4096, 10, 512, True), (3, 3, 7, False)])
def test_dispatch_bitwise(torch, T, k, E, zipf):
    say(f"case: dispatch T={T} k={k} E={E} zipf={zipf}")
    logits = O.gen_normal(5, T, T * E).reshape(T, E)
    if zipf:
        logits = logits + S.zipf_bias(E, 1.2, 5, n_tokens=T, top_k=k, n_embd=1, w_sigma=1.0)[None, :]
    ids, _ = O.route_dev(logits, k)
    counts, offsets, perm, slot = S.dispatch(dev(torch, ids), E)
    want = O.dispatch(ids, E)
    for got, w_ in zip((counts, offsets, perm, slot), want):
        assert np.array_equal(host(torch, got), w_)


def test_dispatch_out_of_range_ids_are_not_dispatched(torch):
    say("case: dispatch out-of-range ids")
    ids = np.array([[0, 1], [5, 1], [9, 0]], np.int32)   # 9 >= E = 6
    counts, offsets, perm, slot = S.dispatch(dev(torch, ids), 6)
    c = host(torch, counts)
    assert c.sum() == 5 and host(torch, slot)[4] == -1   # pair 4 = (token 2, slot 0) has id 9


# ------------------------------------------------------------------------------------------------ the whole block

_LAYERS = {}


def layer(torch, g, seed, bias=None):
    key = (tuple(vars(g).values()), seed, None if bias is None else bias.tobytes())
    if key not in _LAYERS:
        _LAYERS.clear()
        w_host = O.make_weights(g, seed, zipf_bias=bias)
        w_dev = S.synth_layer(S.Geom(**vars(g)), seed,
                              logit_bias=None if bias is None else dev(torch, bias))
        _LAYERS[key] = (w_host, w_dev)
    return _LAYERS[key]


CASES = [
    # name, geometry, T, seed, add_shared
    ("golden small", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4), 3, 4242, True),
    ("config 1 (decode b=1)", {}, 1, 1, True),
    ("config 2 (decode b=16)", {}, 16, 2, True),
    ("decode b=64", {}, 64, 3, True),
    ("reference model shape H=2560 F=640", dict(n_embd=2560, n_ff=640, n_ff_shared=640, n_expert=64), 4, 5, True),
    ("no shared expert", dict(sh_type=-1, n_expert=64), 5, 6, True),
    ("shared not added", dict(n_expert=64), 5, 7, False),
    ("7 experts top-3", dict(n_embd=256, n_ff=256, n_ff_shared=128, n_expert=7, top_k=3), 9, 8, True),
    ("k = 1, E = 1", dict(n_embd=128, n_ff=128, n_ff_shared=256, n_expert=1, top_k=1), 2, 9, True),
    # the shared down rows are packed more densely per wave than the routed ones: the grid must cover all H rows
    ("shared wider than routed, H=2048", dict(n_embd=2048, n_ff=256, n_ff_shared=512, n_expert=32, top_k=4), 5, 10,
     True),
    # 3200 pairs: the dispatch runs as chunk histograms, one scan and chunk ranks
    ("many pairs, top-32", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=128, top_k=32), 100, 17, True),
    # batches of at most 4 tokens run as the router plus one fused launch (gate/up and down-with-combine
    # work-groups exchanging h through tagged words): its variants
    ("fused, no shared expert, T=2", dict(sh_type=-1, n_expert=64), 2, 21, True),
    ("fused, shared not added, T=4", {}, 4, 22, False),
    ("fused, 96 pairs (the down work-groups' LDS dispatch)",
     dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=128, top_k=32), 3, 23, True),
    ("fused, shared wider than routed, T=3", dict(n_embd=2048, n_ff=256, n_ff_shared=512, n_expert=32, top_k=4), 3,
     24, True),
    # more than 512 experts: 16 logits per lane in the selection (the fused launch's one-token and small-batch
    # routes, and k_topk beyond 4 tokens), a non-power-of-two count with a partly filled last logit column
    ("fused, 1024 experts, T=1", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=1024, top_k=8), 1, 25, True),
    ("fused, 1024 experts, T=3", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=1024, top_k=8), 3, 26, True),
    ("600 experts top-10, T=16", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=600, top_k=10), 16, 27, True),
    # wider intermediate rows: the fused launch at n_ff 1024; at n_ff 2048 its down rows would take more than two
    # units per lane, so the small batch runs as the three-launch path
    ("n_ff 1024, T=1", dict(n_embd=1024, n_ff=1024, n_ff_shared=1024, n_expert=64, top_k=8), 1, 28, True),
    ("n_ff 2048, T=2", dict(n_embd=512, n_ff=2048, n_ff_shared=2048, n_expert=32, top_k=4), 2, 29, True),
    ("n_ff 2048, b=16", dict(n_embd=512, n_ff=2048, n_ff_shared=2048, n_expert=32, top_k=4), 16, 30, True),
    # the f32 router of the literal configs[0] (router_dtype 1): f32 weights and activations in the router
    ("f32 router, config 1 (decode b=1)", dict(router_dtype=1), 1, 41, True),
    ("f32 router, fused T=3", dict(router_dtype=1, n_expert=64), 3, 42, True),
    ("f32 router, b=16", dict(router_dtype=1, n_expert=64), 16, 43, True),
    ("f32 router, H=4096", dict(router_dtype=1, n_embd=4096, n_ff=256, n_ff_shared=256, n_expert=16, top_k=4), 5, 44,
     True),
    ("f32 router, 70 tokens in tiles of 16", dict(router_dtype=1, n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16,
                                                  top_k=4), 70, 45, True),
    ("f32 router, no shared expert", dict(router_dtype=1, sh_type=-1, n_expert=64), 2, 46, True),
    # the f32 router of 4096 values at a small batch (its widest tile in the fused launch's stage of the router)
    ("f32 router, H=4096, T=2",
     dict(router_dtype=1, n_embd=4096, n_ff=256, n_ff_shared=256, n_expert=16, top_k=4), 2, 47, True),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_forward_decode_parity(torch, case):
    name, gkw, T, seed, add_shared = CASES[case]
    say(f"case: forward {name} T={T}")
    g = O.Geom(**gkw)
    w_host, w_dev = layer(torch, g, seed)
    x = O.gen_normal(seed, 100, T * g.n_embd).reshape(T, g.n_embd)
    if name == "golden small":
        f = np.load(os.path.join(GOLD, "layer_small.npz"))
        assert np.array_equal(bits(x), bits(f["x"]))
    ml = S.MoELayer(S.Geom(**vars(g)), w_dev, max_tokens=T)
    yg = guarded(torch, T * g.n_embd, torch.float32)
    yv = yg[:T * g.n_embd].view(T, g.n_embd)
    _, tr = ml.forward(dev(torch, x), y=yv, add_shared=add_shared, trace=True)
    got = host(torch, yg)
    assert (got[T * g.n_embd:] == 7.0).all(), "guard words past y were written"
    y = got[:T * g.n_embd].reshape(T, g.n_embd)
    want, wtr = O.moe_decode_dev(g, w_host, x, add_shared=add_shared, trace=True, n_threads=8)
    for k in ("logits", "ids", "weights", "counts", "offsets", "perm", "slot"):
        a = host(torch, tr[k])
        assert np.array_equal(bits(a), bits(wtr[k])), k
    if g.sh_type >= 0:
        assert np.array_equal(bits(host(torch, tr["sgate"])), bits(wtr["sgate"]))
    assert np.array_equal(bits(y), bits(want)), f"max rel {O.rel_l1_rows(y, want).max()}"
    # the reference's own checks: host routing on the device logits, and the reference-order chain
    ids_r, w_r = O.route_ref(host(torch, tr["logits"]), g.top_k)
    if not np.array_equal(ids_r, host(torch, tr["ids"])) and g.top_k < g.n_expert:
        st, _ = S.router_margin(tr["logits"], g.top_k)  # the diagnostic beside the mismatch
        pytest.fail(f"ids differ from the reference routing; smallest k-th/(k+1)-th margin "
                    f"{host(torch, st)[:, 0].min():.3e}")
    assert np.array_equal(ids_r, host(torch, tr["ids"]))
    assert np.max(np.abs(host(torch, tr["weights"]) - w_r) / np.abs(w_r)) <= 1e-5
    # north_star's 1e-3 per row against the reference-order chain; a row beyond it (the two orders round an h value
    # to neighbouring q8_1 steps) passes only through the reference's stage-wise check on the device's own stages
    SW.reference_order_gate(g, w_host, x, y, add_shared, lambda: stage_pass(torch, ml, x, add_shared), say)
    if name == "golden small":
        assert np.array_equal(bits(y), bits(f["y"]))
    # determinism: a repeat is bitwise identical
    y2 = ml.forward(dev(torch, x), add_shared=add_shared)
    assert np.array_equal(bits(host(torch, y2)), bits(y))


@pytest.mark.parametrize("router_dtype,T", [(0, 1), (1, 1), (0, 3), (1, 2)])
def test_forward_decode_with_logit_bias(torch, router_dtype, T):
    """A router logit bias (the Zipf-biased routing of the prefill benchmark) at one token, where the router reads x
    straight into registers (bf16 and f32 routers), and in the fused small batch: bitwise the oracle's device order,
    and the routing is the biased one (the bias moves the selection)."""
    say(f"case: logit bias, router_dtype={router_dtype} T={T}")
    g = O.Geom(router_dtype=router_dtype, n_expert=64)
    bias = S.zipf_bias(g.n_expert, 1.2, 7, n_tokens=16, top_k=g.top_k, n_embd=g.n_embd, w_sigma=0.02)
    w_host, w_dev = layer(torch, g, 61 + router_dtype, bias=bias)
    x = O.gen_normal(62, 100, T * g.n_embd).reshape(T, g.n_embd)
    ml = S.MoELayer(S.Geom(**vars(g)), w_dev, max_tokens=T)
    y, tr = ml.forward(dev(torch, x), add_shared=True, trace=True)
    want, wtr = O.moe_decode_dev(g, w_host, x, add_shared=True, trace=True, n_threads=8)
    for k in ("logits", "ids", "weights"):
        assert np.array_equal(bits(host(torch, tr[k])), bits(wtr[k])), k
    assert np.array_equal(bits(host(torch, y)), bits(want))
    unbiased = O.moe_decode_dev(g, O.make_weights(g, 61 + router_dtype), x, add_shared=True, trace=True,
                                n_threads=8)[1]
    assert not np.array_equal(unbiased["ids"], wtr["ids"]), "the bias must change the selection"


STAGE_CASES = [
    # name, geometry, T, seed, add_shared: the expert stages of the trace (FfnTrace's exq, ehq, edown, shared)
    ("stages, config 1 (decode b=1)", {}, 1, 51, True),
    ("stages, small batch T=3 (the fused launch's stages)", dict(n_expert=64), 3, 52, True),
    ("stages, b=16, shared not added", dict(n_expert=64), 16, 53, False),
    ("stages, no shared expert", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4, sh_type=-1), 5, 54,
     True),
    ("stages, IQ2_S", dict(n_embd=512, n_ff=512, n_ff_shared=512, n_expert=16, top_k=4, w_type=22, sh_type=22), 6, 55,
     True),
]


@pytest.mark.parametrize("case", range(len(STAGE_CASES)))
def test_forward_trace_stages_bitwise(torch, case):
    """A traced call with the expert stages: xq, hq, parts and shared bitwise against the oracle's own trace; y
    bitwise the same as the untraced call (the fused small-batch launch when it applies) and the oracle's."""
    name, gkw, T, seed, add_shared = STAGE_CASES[case]
    say(f"case: forward {name}")
    g = O.Geom(**gkw)
    w_host, w_dev = layer(torch, g, seed)
    x = O.gen_normal(seed, 100, T * g.n_embd).reshape(T, g.n_embd)
    ml = S.MoELayer(S.Geom(**vars(g)), w_dev, max_tokens=T)
    y_plain = host(torch, ml.forward(dev(torch, x), add_shared=add_shared))
    y, tr = ml.forward(dev(torch, x), add_shared=add_shared, trace=True, stages=True)
    want, wtr = O.moe_decode_dev(g, w_host, x, add_shared=add_shared, trace=True, n_threads=8)
    assert np.array_equal(bits(host(torch, y)), bits(want))
    assert np.array_equal(bits(y_plain), bits(want))
    assert np.array_equal(host(torch, tr["xq"]).ravel(), wtr["xq"].ravel()), "xq"
    assert np.array_equal(host(torch, tr["hq"]).ravel(), wtr["hq"].ravel()), "hq"
    assert np.array_equal(bits(host(torch, tr["parts"])), bits(wtr["parts"])), "parts"
    if g.sh_type >= 0:
        assert np.array_equal(bits(host(torch, tr["shared"])), bits(wtr["shared"])), "shared"
    assert host(torch, tr["overflow"])[0] == 0
    # the gate and up dots are the ones h was formed from: SwiGLU + q8_1 of them is the device's h, bit for bit
    htr = {k: host(torch, v) for k, v in tr.items()}
    assert np.array_equal(O.swiglu_q8(htr["egate"], htr["eup"]), htr["hq"].ravel()), "egate/eup vs hq"
    if g.sh_type >= 0:
        Fs = g.n_ff_shared
        sgu = htr["sgu"].reshape(2, T, -1)[:, :, :Fs]
        assert np.array_equal(O.swiglu_q8(sgu[0], sgu[1]), htr["shq"].reshape(T, -1)[:, :Fs // 32 * 36].ravel())
    # the reference's stage-wise check (walk_ffn): every stage from the device's own inputs, in the reference's
    # order, within 1e-5
    rep = SW.stagewise(g, w_host, x, htr, host(torch, y), add_shared)
    say(f"  stage-wise: {rep.summary()}")
    assert rep.ok(), rep.summary()


@pytest.mark.parametrize("T,E,K", [(37, 512, 10), (5, 1000, 1), (4, 64, 63), (3, 100, 7)])
def test_router_margin_bitwise(torch, T, E, K):
    """The router-margin diagnostic (smoe_router_margin) bitwise against the oracle's device order, including rows
    of exact ties."""
    say(f"case: router margin T={T} E={E} k={K}")
    l = (O.gen_normal(T + E, 7, T * E) * 0.9).reshape(T, E)
    l[0] = 0.25                       # all equal: ids k-1, k, margin 0
    if T > 2:
        l[1, :12] = l[1].max() + 1.0  # a 12-way tie at the top
    st, ids = S.router_margin(dev(torch, l), K)
    wst, wids = O.router_margin_dev(l, K)
    assert np.array_equal(host(torch, ids), wids)
    assert np.array_equal(bits(host(torch, st)), bits(wst))


def test_forward_zero_tokens_and_refusals_leave_output(torch):
    say("case: forward zero tokens / refusals")
    g = S.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4)
    w = S.synth_layer(g, 1)
    ml = S.MoELayer(g, w, max_tokens=4)
    y = torch.full((4, 256), 7.0, device="cuda")
    x = torch.zeros((0, 256), device="cuda")
    ml.forward(x, y=y)
    assert (host(torch, y) == 7.0).all()
    small = S.MoELayer(g, w, max_tokens=1)
    with pytest.raises(S.SmoeError):
        small.forward(torch.zeros((4, 256), device="cuda"), y=y)
    import ctypes as C
    x4 = torch.zeros(256 * 4, device="cuda")
    st = S.lib().smoe_forward(C.byref(g.c()), C.byref(S._weights_c(w)), x4.data_ptr(), 4, y.data_ptr(), 1,
                              small.ws.data_ptr(), small.ws_bytes, None, S._stream())
    assert st == -2
    assert (host(torch, y) == 7.0).all()


@pytest.mark.parametrize("rows,n,with_r,inplace", [(16, 2048, True, False), (3, 2560, True, True), (5, 300, False, False),
                                                   (1, 4096, True, False)])
def test_residual_rmsnorm_bitwise(torch, rows, n, with_r, inplace):
    say(f"case: residual_rmsnorm rows={rows} n={n} r={with_r} inplace={inplace}")
    x = O.gen_normal(9, n, rows * n).reshape(rows, n)
    r = O.gen_normal(9, n + 7, rows * n).reshape(rows, n) if with_r else None
    xd = dev(torch, x)
    out = S.residual_rmsnorm(xd, None if r is None else dev(torch, r), 1e-6, out=xd if inplace else None)
    assert np.array_equal(bits(host(torch, out)), bits(O.residual_rmsnorm_dev(x, r, 1e-6)))


def test_layer_binding_refuses_bad_tensors(torch):
    """MoELayer.forward / forward_residual refuse a float16, non-contiguous, narrower or host tensor (x or y)
    before any launch; y keeps its contents."""
    say("case: binding refusals")
    g = S.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4)
    layer = S.MoELayer(g, S.synth_layer(g, 3), max_tokens=4)
    x = torch.zeros((2, 256), dtype=torch.float32, device="cuda")
    y = torch.full((2, 256), 7.0, device="cuda")
    bad_x = [x.half(), torch.zeros((256, 2), device="cuda").t(), x[:, :128].contiguous(), x.cpu(), x[0]]
    for bx in bad_x:
        with pytest.raises(S.SmoeError):
            layer.forward(bx, y)
    for by in (y.half(), y[:, :128].contiguous(), y.cpu(), y.t()):
        with pytest.raises(S.SmoeError):
            layer.forward(x, by)
    with pytest.raises(S.SmoeError):
        layer.forward_residual(x.half(), x, torch.empty_like(x), y)
    with pytest.raises(S.SmoeError):
        layer.forward_residual(x, x[:1], torch.empty_like(x), y)
    assert bool((host(torch, y) == 7.0).all())
