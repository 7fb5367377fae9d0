"""GPU parity of the layer call's hyper-connection ends (smoe_hc_read / smoe_hc_write, gr_read / gr_write of
FfnExec::run, metal/include/strata/metal/gr.hpp:44-48) and of the whole call smoe_ffn_run, through the C ABI,
against the oracle on the same seeded inputs: bitwise against its device-order restatement (or_hc_read_dev,
or_hc_write_dev, then or_moe_decode_dev / or_moe_prefill for the block), and within the reference's own 1e-4 rel_l1
(metal/src/gr_parity.cpp) against its float64-accumulated reference order.  Guard words past every output stay put,
refused calls write nothing."""
import ctypes as C
import sys

import numpy as np
import pytest

import oracle as O
import stratametal_amd as S

pytestmark = pytest.mark.gpu
GUARD = 16
FAKE = 0x10000000


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


def rel_l1(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return np.abs(a - b).sum() / max(np.abs(b).sum(), 1e-30)


def hc_dev(torch, w, n):
    return S.HyperConnection(n, w.hc, w.hc_lr, dev(torch, w.norm), dev(torch, w.down.view(np.int16)),
                             dev(torch, w.up.view(np.int16)), dev(torch, w.inject.view(np.int16)), eps=w.eps)


def streams(seed, T, hc, n):
    R = O.gen_normal(seed, 41, T * hc * n).reshape(T, hc, n)
    return (R * (3.0 ** np.arange(hc, dtype=np.float32))[None, :, None]).astype(np.float32)


READ_CASES = [
    # n_embd, hc, hc_lr, T
    (2048, 4, 320, 1),   # the reference model's ends at decode b=1
    (2048, 4, 320, 5),
    (256, 4, 32, 3),
    (512, 2, 64, 2),
    (1024, 8, 128, 2),   # eight streams: every wave of the mix kernel takes two rows
    (4096, 4, 2048, 1),  # the largest activation stage (hc * n_embd = 16384) and low-rank width
    (8, 1, 8, 4),
    (72, 3, 24, 3),      # ragged: no multiple of 64 anywhere
]


@pytest.mark.parametrize("case", range(len(READ_CASES)))
def test_hc_read_parity(torch, case):
    n, hc, hc_lr, T = READ_CASES[case]
    say(f"case: hc_read n={n} hc={hc} hc_lr={hc_lr} T={T}")
    w = O.make_hc(n, hc, hc_lr, 100 + case)
    R = streams(case, T, hc, n)
    H = hc_dev(torch, w, n)
    mg = torch.full((T * n + GUARD,), 7.0, dtype=torch.float32, device="cuda")
    ig = torch.full((T * hc + GUARD,), 7.0, dtype=torch.float32, device="cuda")
    H.read(dev(torch, R), mixed=mg[:T * n], inject=ig[:T * hc])
    m, i = host(torch, mg), host(torch, ig)
    assert (m[T * n:] == 7.0).all() and (i[T * hc:] == 7.0).all(), "guard words written"
    m, i = m[:T * n].reshape(T, n), i[:T * hc].reshape(T, hc)
    want_m, want_i = O.hc_read_dev(R, n, w)
    assert np.array_equal(bits(m), bits(want_m)), f"mixed rel_l1 {rel_l1(m, want_m):.3e}"
    assert np.array_equal(bits(i), bits(want_i)), f"inject rel_l1 {rel_l1(i, want_i):.3e}"
    ref_m, ref_i = O.hc_read_ref(R, n, w)
    assert rel_l1(m, ref_m) <= 1e-4 and rel_l1(i, ref_i) <= 1e-4


def test_hc_read_without_inject_and_repeat(torch):
    say("case: hc_read, inject NULL (the final mixer)")
    n, hc, hc_lr, T = 256, 4, 32, 2
    w = O.make_hc(n, hc, hc_lr, 7)
    R = streams(7, T, hc, n)
    H = hc_dev(torch, w, n)
    mixed = torch.empty((T, n), dtype=torch.float32, device="cuda")
    ws = torch.empty(S.lib().smoe_hc_read_workspace_bytes(C.byref(H._c), n, T), dtype=torch.uint8, device="cuda")
    Rd = dev(torch, R)
    S._check(S.lib().smoe_hc_read(C.byref(H._c), n, Rd.data_ptr(), T, mixed.data_ptr(), None, ws.data_ptr(),
                                  ws.numel(), S._stream()))
    want_m, _ = O.hc_read_dev(R, n, w)
    assert np.array_equal(bits(host(torch, mixed)), bits(want_m))
    m2, _ = H.read(Rd)
    assert np.array_equal(bits(host(torch, m2)), bits(want_m))
    assert np.array_equal(host(torch, Rd), R), "the read wrote its input"


@pytest.mark.parametrize("n,hc,T", [(2048, 4, 3), (72, 3, 5), (8, 1, 1)])
def test_hc_write_parity(torch, n, hc, T):
    say(f"case: hc_write n={n} hc={hc} T={T}")
    R = streams(n, T, hc, n)
    y = O.gen_normal(n, 51, T * n).reshape(T, n)
    inj = (O.gen_normal(n, 52, T * hc) * 4.0).reshape(T, hc).astype(np.float32)
    want = O.hc_write_dev(R, y, inj, n, hc)
    H = hc_dev(torch, O.make_hc(n, hc, 8, n), n)  # the write reads only hc and n_embd of it
    og = torch.full((T * hc * n + GUARD,), 7.0, dtype=torch.float32, device="cuda")
    H.write(dev(torch, R), dev(torch, y), dev(torch, inj), out=og[:T * hc * n])
    got = host(torch, og)
    assert (got[T * hc * n:] == 7.0).all()
    assert np.array_equal(bits(got[:T * hc * n].reshape(T, hc, n)), bits(want))
    Rd = dev(torch, R)  # in place
    H.write(Rd, dev(torch, y), dev(torch, inj), out=Rd)
    assert np.array_equal(bits(host(torch, Rd)), bits(want))


FFN_CASES = [
    # name, geometry, hc, hc_lr, T, seed, add_shared
    ("decode b=1, reference ends", dict(n_expert=64), 4, 320, 1, 31, True),
    ("decode b=3 fused block, shared not added", dict(n_expert=64), 4, 320, 3, 32, False),
    ("decode b=16", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4), 4, 32, 16, 33, True),
    ("prefill 160 tokens (MFMA block)", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4), 2, 64,
     160, 34, True),
]


@pytest.mark.parametrize("case", range(len(FFN_CASES)))
def test_ffn_run_parity(torch, case):
    name, gkw, hc, hc_lr, T, seed, add_shared = FFN_CASES[case]
    say(f"case: ffn_run {name}")
    g = O.Geom(**gkw)
    n = g.n_embd
    w_host = O.make_weights(g, seed)
    w_dev = S.synth_layer(S.Geom(**vars(g)), seed)
    hw = O.make_hc(n, hc, hc_lr, seed)
    R = streams(seed, T, hc, n)
    layer = S.FfnLayer(S.Geom(**vars(g)), w_dev, hc_dev(torch, hw, n), max_tokens=T)
    og = torch.full((T * hc * n + GUARD,), 7.0, dtype=torch.float32, device="cuda")
    Rd = dev(torch, R)
    layer.run(Rd, out=og[:T * hc * n], add_shared=add_shared)
    got = host(torch, og)
    assert (got[T * hc * n:] == 7.0).all(), "guard words past out were written"
    got = got[:T * hc * n].reshape(T, hc, n)
    mixed, inj = O.hc_read_dev(R, n, hw)
    if T >= S.MFMA_TOKENS:
        # the prefill path's router runs on the matrix cores (logits within ~1e-7 of the exact dot): with every
        # token's k-th / (k+1)-th logit gap far above that, its routing is the oracle's
        y, otr = O.moe_prefill(g, w_host, mixed, add_shared=add_shared, trace=True, n_threads=16)
        top = -np.sort(-otr["logits"], axis=1)
        gap = (top[:, g.top_k - 1] - top[:, g.top_k]) / np.abs(otr["logits"]).max(axis=1)
        assert gap.min() > 1e-4, f"a token sits at a routing tie ({gap.min():.2e}): choose another seed"
        want = O.hc_write_dev(R, y, inj, n, hc)
        # the block's prefill contract holds per row within 1e-3 of the oracle; the write adds it to the streams
        yg = (got - R) / (2.0 / (1.0 + np.exp(-inj.astype(np.float64) / hc)))[:, :, None]
        assert O.rel_l1_rows(yg[:, 0, :].astype(np.float32), y).max() <= 1e-3
        assert rel_l1(got, want) <= 1e-3
    else:
        y = O.moe_decode_dev(g, w_host, mixed, add_shared=add_shared, n_threads=16)
        want = O.hc_write_dev(R, y, inj, n, hc)
        assert np.array_equal(bits(got), bits(want)), f"rel_l1 {rel_l1(got, want):.3e}"
    # in place (out = residual), repeated: the same bits
    layer.run(Rd, out=Rd, add_shared=add_shared)
    assert np.array_equal(bits(host(torch, Rd)), bits(got))


def test_hc_refusals_write_nothing(torch):
    say("case: hc refusals")
    L = S.lib()
    n, hc, hc_lr, T = 256, 4, 32, 2
    w = O.make_hc(n, hc, hc_lr, 3)
    H = hc_dev(torch, w, n)
    Rd = dev(torch, streams(3, T, hc, n))
    mixed = torch.full((T, n), 7.0, dtype=torch.float32, device="cuda")
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    need = L.smoe_hc_read_workspace_bytes(C.byref(H._c), n, T)
    assert 0 < need < (1 << 20)
    bad = [S._Hc(hc, 36, 1e-6, *[t.data_ptr() for t in H.tensors]),       # hc_lr not a multiple of 8
           S._Hc(9, hc_lr, 1e-6, *[t.data_ptr() for t in H.tensors]),     # more than 8 streams
           S._Hc(hc, hc_lr, -1.0, *[t.data_ptr() for t in H.tensors]),    # negative eps
           S._Hc(hc, hc_lr, 1e-6, None, *[t.data_ptr() for t in H.tensors[1:]])]
    for h in bad:
        assert L.smoe_hc_read(C.byref(h), n, Rd.data_ptr(), T, mixed.data_ptr(), None, ws.data_ptr(), ws.numel(),
                              S._stream()) != 0
    assert L.smoe_hc_read(C.byref(H._c), 252, Rd.data_ptr(), T, mixed.data_ptr(), None, ws.data_ptr(), ws.numel(),
                          S._stream()) != 0  # n_embd not a multiple of 8
    assert L.smoe_hc_read(C.byref(H._c), n, Rd.data_ptr(), T, mixed.data_ptr(), None, ws.data_ptr(), need - 1,
                          S._stream()) == -2
    assert L.smoe_hc_read(C.byref(H._c), n, Rd.data_ptr() + 2, T, mixed.data_ptr(), None, ws.data_ptr(), ws.numel(),
                          S._stream()) == -5
    assert L.smoe_hc_read(C.byref(H._c), n, Rd.data_ptr(), 0, mixed.data_ptr(), None, ws.data_ptr(), ws.numel(),
                          S._stream()) == 0
    assert (host(torch, mixed) == 7.0).all()
    # the whole call: a block the forward call refuses stops it before gr_read
    g = S.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4)
    lay = S.FfnLayer(g, S.synth_layer(g, 1), H, max_tokens=T)
    out = torch.full((T, hc, n), 7.0, dtype=torch.float32, device="cuda")
    wc = S._Weights(*([FAKE] * 3 + [None] + [FAKE] * 4 + [None]))  # the router missing
    assert L.smoe_ffn_run(C.byref(lay._gc), C.byref(wc), C.byref(H._c), Rd.data_ptr(), T, out.data_ptr(), 1,
                          lay.ws.data_ptr(), lay.ws_bytes, None, S._stream()) == -6
    assert L.smoe_ffn_run(C.byref(lay._gc), C.byref(lay._wc), C.byref(H._c), Rd.data_ptr(), T, out.data_ptr(), 1,
                          lay.ws.data_ptr(), lay.ws_bytes - 1, None, S._stream()) == -2
    assert (host(torch, out) == 7.0).all()
    with pytest.raises(S.SmoeError):
        S.FfnLayer(S.Geom(n_embd=512, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4), lay.w, H, max_tokens=T)
