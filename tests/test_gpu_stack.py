"""The stacked configuration (x_{l+1} = RMSNorm(x_l + MoE_l(x_l)), unit weight, eps 1e-6,
over seeded layers) on a small stack through the C ABI: the decode contract bit for bit against the oracle's
chain (or_moe_decode_dev, or_residual_rmsnorm_dev); the prefill contract layer by layer on the GPU's own layer
inputs, routing exact and each layer within 1e-3 per row of or_moe_prefill, the junction bit for bit."""
import sys

import numpy as np
import pytest

import oracle as O
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
        want, wtr = O.moe_prefill(g, hostw[l], xg, add_shared=True, trace=True, n_threads=16)
        assert np.array_equal(host(torch, tr["ids"]).reshape(-1), np.asarray(wtr["ids"]).reshape(-1)), l
        err = O.rel_l1_rows(host(torch, y), want)
        say(f"  layer {l}: max rel_l1 {err.max():.3e}")
        assert err.max() <= 1e-3
        yg = host(torch, y)
        xd = S.residual_rmsnorm(xd, y, EPS)
        assert np.array_equal(bits(host(torch, xd)), bits(O.residual_rmsnorm_dev(xg, yg, EPS))), l
