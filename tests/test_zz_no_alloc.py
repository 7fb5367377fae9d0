"""GPU test of smoe_forward_static, the entry point that allocates nothing (the library's static device
scratch instead of a caller workspace): its output equals smoe_forward's bit for bit on consecutive calls on the
same GPU, each smaller than the one before (so a call finds the previous call's contents in the scratch), on
both contracts (MFMA from 128 tokens, the GEMV batch path, the small-batch path)."""
import ctypes as C

import numpy as np
import pytest
import torch

import stratametal_amd as S

pytestmark = pytest.mark.gpu


def _static(g, w, x, y, add_shared=1):
    L = S.lib()
    st = L.smoe_forward_static(C.byref(g.c()), C.byref(S._weights_c(w)), x.data_ptr(), x.shape[0], y.data_ptr(),
                               add_shared, None, S._stream())
    S._check(st)
    return y


@pytest.mark.parametrize("wtype", [S.Q2_0, S.IQ2_S])
def test_forward_static_matches_forward(wtype):
    g = S.Geom(w_type=wtype, sh_type=wtype)
    w = S.synth_layer(g, 777 + wtype)
    sizes = (200, 16, 3, 1) if wtype == S.Q2_0 else (64, 5, 1)
    layer = S.MoELayer(g, w, max_tokens=max(sizes))
    for i, T in enumerate(sizes):
        print(f"static vs forward: type {wtype}, call {i}, {T} tokens", flush=True)
        x = S.synth_normal(900 + i, 100 + wtype, T * g.n_embd).view(T, g.n_embd)
        want = layer.forward(x)
        got = _static(g, w, x, torch.full_like(x, float("nan")))
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32)), (wtype, T)


def test_forward_static_refuses_oversize_batch():
    g = S.Geom()
    w = S.synth_layer(g, 5)
    T = 400
    x = torch.zeros((T, g.n_embd), dtype=torch.float32, device="cuda")
    y = torch.full_like(x, 7.0)
    with pytest.raises(S.SmoeError) as e:
        _static(g, w, x, y)
    assert e.value.status == -2
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())  # a refused call writes nothing
