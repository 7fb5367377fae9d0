"""The stacked configuration (x_{l+1} = RMSNorm(x_l + MoE_l(x_l)), unit weight, eps 1e-6,
over seeded layers) on a small stack through the C ABI: the decode contract bit for bit against the oracle's
chain (or_moe_decode_dev, or_residual_rmsnorm_dev); the prefill contract layer by layer on the GPU's own layer
inputs, routing exact and each layer within 1e-3 per row of or_moe_prefill, the junction bit for bit; the fused
junction (smoe_forward_residual) bit for bit against the junction and the call made apart."""
import sys

import numpy as np
import pytest

import oracle as O
import prefill_check as PC
import stratametal_amd as S

pytestmark = pytest.mark.gpu
GEOM = dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4)
N_LAYERS = 3
EPS = 1e-6


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
    return np.ascontiguousarray(a).view(np.uint32)


def stack(torch, T):
    g = O.Geom(**GEOM)
    hostw = [O.make_weights(g, 700 + l) for l in range(N_LAYERS)]
    layers = [S.MoELayer(S.Geom(**GEOM), S.synth_layer(S.Geom(**GEOM), 700 + l), max_tokens=T) for l in range(N_LAYERS)]
    return g, hostw, layers


def test_stack_decode_chain_bitwise(torch):
    say("case: stack of 3, decode T=5")
    T = 5
    g, hostw, layers = stack(torch, T)
    x = O.gen_normal(77, 100, T * g.n_embd).reshape(T, g.n_embd)
    xd, xh = dev(torch, x), x
    for l in range(N_LAYERS):
        y = layers[l].forward(xd, add_shared=True, path=S.PATH_GEMV)
        xd = S.residual_rmsnorm(xd, y, EPS)
        yh = O.moe_decode_dev(g, hostw[l], xh, add_shared=True)
        assert np.array_equal(bits(host(torch, y)), bits(yh)), f"layer {l} MoE"
        xh = O.residual_rmsnorm_dev(xh, yh, EPS)
        assert np.array_equal(bits(host(torch, xd)), bits(xh)), f"layer {l} junction"


def test_stack_prefill_layers_on_gpu_inputs(torch):
    say("case: stack of 3, prefill T=130")
    T = 130
    g, hostw, layers = stack(torch, T)
    xd = dev(torch, O.gen_normal(78, 100, T * g.n_embd).reshape(T, g.n_embd))
    for l in range(N_LAYERS):
        xg = host(torch, xd)
        y, tr = layers[l].forward(xd, add_shared=True, trace=True, path=S.PATH_MFMA)
        htr = {k: host(torch, v) for k, v in tr.items()}
        PC.router_stagewise(g, hostw[l], xg, htr)
        want = PC.prefill_want(g, hostw[l], xg, htr, add_shared=True, n_threads=16)
        err = O.rel_l1_rows(host(torch, y), want)
        say(f"  layer {l}: max rel_l1 {err.max():.3e}")
        assert err.max() <= 1e-3
        yg = host(torch, y)
        xd = S.residual_rmsnorm(xd, y, EPS)
        assert np.array_equal(bits(host(torch, xd)), bits(O.residual_rmsnorm_dev(xg, yg, EPS))), l


FUSED = [  # T, geometry, path the call takes
    (1, GEOM, "GEMV, one token (fused into the routing gu kernel's router)"),
    (3, GEOM, "GEMV, small batch"),
    (5, GEOM, "GEMV, routed through the dispatch"),
    (100, GEOM, "GEMV, token tiles of 16"),
    (130, GEOM, "MFMA (junction kernel, then the call)"),
    (1, {}, "GEMV, the bench geometry"),
    (4, dict(n_embd=2560, n_ff=640, n_ff_shared=640, n_expert=64), "GEMV, H=2560"),
    # the f32 router (router_dtype 1): the junction stages f32 values
    (1, dict(router_dtype=1), "GEMV, f32 router, the bench geometry"),
    (100, dict(GEOM, router_dtype=1), "GEMV, f32 router, token tiles"),
    (130, dict(GEOM, router_dtype=1), "MFMA, f32 router"),
]


@pytest.mark.parametrize("case", range(len(FUSED)))
def test_fused_junction_matches_separate_calls(torch, case):
    T, gkw, what = FUSED[case]
    say(f"case: fused junction T={T} {gkw or 'default'} ({what})")
    g = S.Geom(**gkw)
    H = g.n_embd
    ml = S.MoELayer(g, S.synth_layer(g, 900 + case), max_tokens=T)
    xp = O.gen_normal(80 + case, 100, T * H).reshape(T, H)
    rp = O.gen_normal(81 + case, 100, T * H).reshape(T, H)
    xpd, rpd = dev(torch, xp), dev(torch, rp)
    x_ref = S.residual_rmsnorm(xpd, rpd, EPS)
    y_ref = ml.forward(x_ref)
    x = torch.full_like(xpd, 7.0)
    y = ml.forward_residual(xpd, rpd, x, eps=EPS)
    assert np.array_equal(bits(host(torch, x)), bits(O.residual_rmsnorm_dev(xp, rp, EPS))), "junction vs oracle"
    assert np.array_equal(bits(host(torch, x)), bits(host(torch, x_ref))), "junction"
    assert np.array_equal(bits(host(torch, y)), bits(host(torch, y_ref))), "layer output"
    # y may be r_prev (the stack's own buffer reuse); x_prev and r_prev are left as they were otherwise
    r2 = rpd.clone()
    x2 = torch.empty_like(xpd)
    ml.forward_residual(xpd, r2, x2, y=r2, eps=EPS)
    assert np.array_equal(bits(host(torch, r2)), bits(host(torch, y_ref)))
    assert np.array_equal(bits(host(torch, x2)), bits(host(torch, x_ref)))
    assert np.array_equal(bits(host(torch, xpd)), bits(xp))


def test_fused_stack_decode_chain_bitwise(torch):
    say("case: stack of 3 with fused junctions, decode T=2")
    T = 2
    g, hostw, layers = stack(torch, T)
    x = O.gen_normal(79, 100, T * g.n_embd).reshape(T, g.n_embd)
    bufs = [dev(torch, x), torch.empty((T, g.n_embd), dtype=torch.float32, device="cuda")]
    y = layers[0].forward(bufs[0], add_shared=True)
    xh = x
    yh = O.moe_decode_dev(g, hostw[0], xh, add_shared=True)
    for l in range(1, N_LAYERS):
        layers[l].forward_residual(bufs[(l - 1) % 2], y, bufs[l % 2], y=y, eps=EPS)
        xh = O.residual_rmsnorm_dev(xh, yh, EPS)
        yh = O.moe_decode_dev(g, hostw[l], xh, add_shared=True)
        assert np.array_equal(bits(host(torch, bufs[l % 2])), bits(xh)), f"layer {l} junction"
        assert np.array_equal(bits(host(torch, y)), bits(yh)), f"layer {l} MoE"
