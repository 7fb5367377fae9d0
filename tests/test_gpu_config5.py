"""BASELINE configs[4] at its own geometry: a stack of Qwen3-Next-style MoE layers (H 2048, 512 Q2_0 experts + a
shared one, top-10, FF 512, seeded N(0, 0.02) routers, no routing bias) chained as x_{l+1} = RMSNorm(x_l +
MoE_l(x_l)) (unit weight, eps 1e-6), through the C ABI.

- One layer on 4096 prefill tokens (the configuration's prefill, SMOE_PATH_AUTO: the MFMA contract, the many-pair
  dispatch): logits, shared gate dots, ids, weights and the dispatch bit for bit against the oracle for every
  token; output rows within 1e-3 rel_l1 of or_moe_prefill on 128 rows spread over the batch (a row depends only on
  its own token, so the oracle runs those rows alone).
- Six layers chained at batch 1 (the configuration's decode) through smoe_forward_residual, bit for bit against the
  oracle's chain (or_moe_decode_dev, or_residual_rmsnorm_dev).
- The fused junction at 4096 tokens bit for bit against the junction and the call made apart.
- All 48 layers on the 4096-token prefill, by properties that hold at any size: every junction row's mean square
  equals ms / (ms + eps) of its input row (within 1e-5), everything stays finite, and a repeat is bit for bit
  the same (the reference's layer walk checks its stack stage by stage in the same spirit:
  metal/src/pack_parity.cpp:8836-8873)."""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle as O
import prefill_check as PC
import stratametal_amd as S

pytestmark = pytest.mark.gpu
EPS = 1e-6
T_PREFILL = 4096
TOL = 1e-3


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


def test_config5_layer_prefill_4096(torch):
    say("case: configs[4] layer, 4096-token prefill")
    g = O.Geom()
    H, E, K = g.n_embd, g.n_expert, g.top_k
    seed = 5001
    w_host = O.make_weights(g, seed)
    w_dev = S.synth_layer(S.Geom(), seed)
    x = O.gen_normal(seed, 100, T_PREFILL * H).reshape(T_PREFILL, H)
    ml = S.MoELayer(S.Geom(), w_dev, max_tokens=T_PREFILL)
    y, tr = ml.forward(dev(torch, x), trace=True)
    yg = host(torch, y)
    assert np.isfinite(yg).all()
    # the router on the matrix cores: every 32nd token's logits within 1e-5 of the exact dot, the routing and the
    # dispatch of every token exactly the device order's of the device's logits
    htr = {k: host(torch, v) for k, v in tr.items()}
    rows = np.arange(0, T_PREFILL, 32)
    worst = PC.router_stagewise(g, w_host, x, htr, rows=rows)
    counts = htr["counts"]
    say(f"  routing exact; logits {worst:.2e} from the exact dot; {int((counts > 0).sum())} experts touched, "
        f"hottest {int(counts.max())} pairs")
    # output rows: every 32nd token through the prefill contract routed from the same logits
    ref = PC.prefill_want(g, w_host, x, htr, rows=rows, n_threads=16)
    err = O.rel_l1_rows(yg[rows], ref)
    say(f"  {len(rows)} rows: max rel_l1 {err.max():.3e} (mean {err.mean():.3e})")
    assert err.max() <= TOL
    # a repeat is bitwise identical
    assert np.array_equal(bits(host(torch, ml.forward(dev(torch, x)))), bits(yg))


def test_config5_decode_chain_of_6_bitwise(torch):
    say("case: configs[4] decode, 6 chained layers at batch 1 (fused junctions)")
    g = O.Geom()
    H = g.n_embd
    n_layers = 6
    seeds = [5100 + l for l in range(n_layers)]
    layers = [S.MoELayer(S.Geom(), S.synth_layer(S.Geom(), s), max_tokens=1) for s in seeds]
    x = O.gen_normal(5200, 100, H).reshape(1, H)
    bufs = [dev(torch, x), torch.empty((1, H), dtype=torch.float32, device="cuda")]
    y = layers[0].forward(bufs[0])
    xh = x
    yh = O.moe_decode_dev(g, O.make_weights(g, seeds[0]), xh)
    assert np.array_equal(bits(host(torch, y)), bits(yh)), "layer 0"
    for l in range(1, n_layers):
        layers[l].forward_residual(bufs[(l - 1) % 2], y, bufs[l % 2], y=y, eps=EPS)
        xh = O.residual_rmsnorm_dev(xh, yh, EPS)
        yh = O.moe_decode_dev(g, O.make_weights(g, seeds[l]), xh)
        assert np.array_equal(bits(host(torch, bufs[l % 2])), bits(xh)), f"layer {l} junction"
        assert np.array_equal(bits(host(torch, y)), bits(yh)), f"layer {l} MoE"
        say(f"  layer {l} bitwise")


def test_config5_fused_junction_4096_matches_separate(torch):
    say("case: configs[4] fused junction at 4096 tokens")
    g = S.Geom()
    H = g.n_embd
    ml = S.MoELayer(g, S.synth_layer(g, 5300), max_tokens=T_PREFILL)
    xp = S.synth_normal(5301, 100, T_PREFILL * H).view(T_PREFILL, H)
    rp = S.synth_normal(5302, 100, T_PREFILL * H).view(T_PREFILL, H)
    x_ref = S.residual_rmsnorm(xp, rp, EPS)
    y_ref = ml.forward(x_ref)
    x = torch.full_like(xp, 7.0)
    y = ml.forward_residual(xp, rp, x, eps=EPS)
    torch.cuda.synchronize()
    assert torch.equal(x.view(torch.int32), x_ref.view(torch.int32)), "junction"
    assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32)), "layer output"


def test_config5_stack_of_48_prefill_properties(torch):
    say("case: configs[4] stack of 48, 4096-token prefill")
    g = S.Geom()
    H, L = g.n_embd, 48
    lib = S.lib()
    weights = [S.synth_layer(g, 6000 + l) for l in range(L)]
    wc = [S._weights_c(w) for w in weights]
    gc = g.c()
    ws_bytes = S.workspace_bytes(g, T_PREFILL)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    x0 = S.synth_normal(6100, 100, T_PREFILL * H).view(T_PREFILL, H)
    xs = [torch.empty_like(x0) for _ in range(2)]
    ys = [torch.empty_like(x0) for _ in range(2)]

    def run(check):
        xs[0].copy_(x0)
        S._check(lib.smoe_forward(C.byref(gc), C.byref(wc[0]), xs[0].data_ptr(), T_PREFILL, ys[0].data_ptr(), 1,
                                  ws.data_ptr(), ws_bytes, None, S._stream()))
        for l in range(1, L):
            xp, yp, xn, yn = xs[(l - 1) % 2], ys[(l - 1) % 2], xs[l % 2], ys[l % 2]
            S._check(lib.smoe_forward_residual(C.byref(gc), C.byref(wc[l]), xp.data_ptr(), yp.data_ptr(),
                                               C.c_float(EPS), xn.data_ptr(), T_PREFILL, yn.data_ptr(), 1,
                                               ws.data_ptr(), ws_bytes, None, S._stream()))
            if check:
                s = xp.double() + yp.double()
                ms_in = (s * s).mean(dim=1)
                ms_out = (xn.double() ** 2).mean(dim=1)
                dev_ = (ms_out - ms_in / (ms_in + EPS)).abs().max().item()
                assert dev_ <= 1e-5, (l, dev_)
                assert bool(torch.isfinite(yn).all()) and bool(torch.isfinite(xn).all()), l
        xl = xs[(L - 1) % 2]
        S.residual_rmsnorm(xl, ys[(L - 1) % 2], EPS, out=xl)
        torch.cuda.synchronize()
        return xl.clone()

    a = run(True)
    assert bool(torch.isfinite(a).all())
    ms = (a.double() ** 2).mean(dim=1)
    assert (ms - 1.0).abs().max().item() <= 1e-5
    b = run(False)
    assert torch.equal(a.view(torch.int32), b.view(torch.int32)), "a repeat of the 48-layer prefill differs"
    say("  48 junctions within 1e-5 of their closed form, finite, repeat bitwise")
