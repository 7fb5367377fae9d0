"""A call's status mask without a trace (smoe_forward_status; SMOE_STATUS_* bits, include/smoe.h).

- The fused decode launches' bounded waits, forced from the host to give up at once (smoe_set_wait_limit(-1): no
  wait polls at all, so every kernel still exits normally): the rows of every down work-group are NaN and the status
  (and a trace's overflow mask) carries SMOE_STATUS_WAIT; with the default bound restored the next call is the
  oracle's bits and its status is 0 (the router launch and the fused launch of the rest, at b=1, a small batch, and
  an f32 router of 4096 values).
- The prefill path's fp16 operand limit: a token whose x reaches 65520 sets SMOE_STATUS_X_FP16 with no trace given.
"""
import sys

import numpy as np
import pytest

import oracle as O
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


def host(torch, t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


CASES = [
    # name, geometry, T
    ("b=1", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4), 1),
    ("T=3", dict(n_embd=512, n_ff=256, n_ff_shared=256, n_expert=32, top_k=4), 3),
    ("f32 router, H 4096",
     dict(router_dtype=1, n_embd=4096, n_ff=256, n_ff_shared=256, n_expert=16, top_k=4), 2),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_wait_give_up_is_reported(torch, case):
    name, gkw, T = CASES[case]
    say(f"case: wait give-up, {name}")
    g = O.Geom(**gkw)
    seed = 80 + case
    w_host = O.make_weights(g, seed)
    w_dev = S.synth_layer(S.Geom(**vars(g)), seed)
    x = O.gen_normal(seed, 100, T * g.n_embd).reshape(T, g.n_embd)
    ml = S.MoELayer(S.Geom(**vars(g)), w_dev, max_tokens=T)
    xd = torch.from_numpy(x).cuda()
    want = O.moe_decode_dev(g, w_host, x)
    y = ml.forward(xd)
    assert np.array_equal(bits(host(torch, y)), bits(want))
    assert int(host(torch, ml.status())[0]) == 0
    assert S.set_wait_limit(-1) > 0
    try:
        y_bad = ml.forward(xd)
        st_bad = ml.status()
        out = dict(overflow=torch.full((1,), -1, dtype=torch.int32, device="cuda"))
        y_tr = torch.empty_like(xd)
        import ctypes as C
        trc = S._Trace(*([None] * 13), out["overflow"].data_ptr())
        S._check(S.lib().smoe_forward_path(C.byref(ml._gc), C.byref(ml._wc), xd.data_ptr(), T, y_tr.data_ptr(), 1,
                                           ml.ws.data_ptr(), ml.ws_bytes, C.byref(trc), 0, S._stream(None)))
        mask_tr = int(host(torch, out["overflow"])[0])
    finally:
        assert S.set_wait_limit(0) == -1
    yb = host(torch, y_bad)
    assert np.isnan(yb).all(), "every down work-group gave up: every row must be NaN"
    assert int(host(torch, st_bad)[0]) == S.STATUS_WAIT
    assert mask_tr == S.STATUS_WAIT
    # the default bound again: the oracle's bits, status 0
    y2 = ml.forward(xd)
    assert np.array_equal(bits(host(torch, y2)), bits(want))
    assert int(host(torch, ml.status())[0]) == 0


def test_prefill_fp16_limit_reported_without_trace(torch):
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4)
    T, seed = 160, 91
    say(f"case: prefill status T={T}")
    w_dev = S.synth_layer(S.Geom(**vars(g)), seed)
    ml = S.MoELayer(S.Geom(**vars(g)), w_dev, max_tokens=T)
    x = O.gen_normal(seed, 100, T * g.n_embd).reshape(T, g.n_embd)
    xd = torch.from_numpy(x).cuda()
    ml.forward(xd, path=S.PATH_MFMA)
    assert int(host(torch, ml.status())[0]) == 0
    x2 = x.copy()
    x2[7, 3] = 1e5  # beyond the fp16 operands of the matrix cores
    ml.forward(torch.from_numpy(x2).cuda(), path=S.PATH_MFMA)
    assert int(host(torch, ml.status())[0]) & S.STATUS_X_FP16
    # a decode-path call on the same workspace reports its own status (no waits gave up)
    ml.forward(xd[:2].contiguous())
    assert int(host(torch, ml.status())[0]) == 0


def test_status_refusals(torch):
    say("case: status refusals")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    junk = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    # (256 bytes into an allocation: never the start of a workspace that a call used)
    assert S.lib().smoe_forward_status(junk.data_ptr() + 256, out.data_ptr(), None) == -1  # no call known there
    assert S.lib().smoe_forward_status(junk.data_ptr(), None, None) == -6
    assert S.lib().smoe_forward_status(junk.data_ptr(), out.data_ptr() + 2, None) == -5
