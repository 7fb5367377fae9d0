"""GPU parity of the IQ2_S (ggml type 22) decode path through the C ABI, against the oracle on the same seeded
inputs: bitwise against the device-order restatement (or_iq2_s_gemv_dev, the block chain or_moe_decode_dev);
within 1e-5 per stage / 1e-3 per row of the reference-order chain (32-lane partials,
metal/shaders/iq.metal:152-180,459-498).  Covers BASELINE configs[3] (batch 64, IQ2_S routed and shared
experts, uniform routing), the stage GEMV at every supported row length, and the refusals of shapes and paths
the IQ2_S kernels do not tile."""
import sys

import numpy as np
import pytest

import oracle as O
import stagewise as SW
import stratametal_amd as S

pytestmark = pytest.mark.gpu
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


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


@pytest.mark.parametrize("n_in,n_out,n_col", [(512, 64, 1), (1024, 96, 2), (2048, 512, 3), (2048, 37, 1)])
def test_mmvq_iq2_s_bitwise(torch, n_in, n_out, n_col):
    say(f"case: mmvq IQ2_S {n_in}x{n_out} cols={n_col}")
    w = O.gen_iq2_s(777, n_in + n_out, n_out * n_in // 256)
    x = O.gen_normal(777, n_col, n_col * n_in)
    xq = O.quant_q8_1(x)
    y = S.mmvq(22, dev(torch, w), dev(torch, xq), n_in, n_out, n_col)
    got = host(torch, y)
    for c in range(n_col):
        xc = xq[c * n_in // 32 * 36:(c + 1) * n_in // 32 * 36]
        assert np.array_equal(bits(got[c]), bits(O.iq2_s_gemv_dev(w, xc, n_in, n_out)))
        assert O.rel_l1_rows(got[c][None], O.iq2_s_gemv_ref(w, xc, n_in, n_out)[None])[0] <= 1e-5


def test_mmvq_iq2_s_odd_block_offset(torch):
    """A byte offset that starts the rows at an odd block (82 bytes, 2 mod 4) is refused as misaligned; an
    even number of blocks in is read exactly."""
    say("case: mmvq IQ2_S byte offset")
    n_in, n_out = 512, 32
    blob = O.gen_iq2_s(5, 5, 2 * n_out * n_in // 256)
    xq = O.quant_q8_1(O.gen_normal(5, 6, n_in))
    off = n_out * n_in // 256 * 82
    y = S.mmvq(22, dev(torch, blob), dev(torch, xq), n_in, n_out, 1, byte_off=off)
    assert np.array_equal(bits(host(torch, y)[0]), bits(O.iq2_s_gemv_dev(blob[off:], xq, n_in, n_out)))
    with pytest.raises(S.SmoeError):
        S.mmvq(22, dev(torch, blob), dev(torch, xq), n_in, n_out, 1, byte_off=82)


CASES = [
    # name, geometry, T, seed, add_shared
    ("config 4 (b=64, IQ2_S, uniform)", dict(w_type=22, sh_type=22), 64, 4, True),
    ("small IQ2_S", dict(n_embd=512, n_ff=512, n_ff_shared=512, n_expert=16, top_k=4, w_type=22, sh_type=22), 5, 41,
     True),
    ("IQ2_S H=1024 no shared", dict(n_embd=1024, n_ff=512, n_expert=32, top_k=6, w_type=22, sh_type=-1), 9, 42, True),
    ("IQ2_S shared not added", dict(n_embd=512, n_ff=1024, n_ff_shared=1024, n_expert=16, top_k=2, w_type=22,
                                    sh_type=22), 3, 43, False),
    ("IQ2_S b=1", dict(w_type=22, sh_type=22), 1, 44, True),
    # 1024 experts in the small-batch route (16 logits per lane), and the widest down rows (n_ff 2048)
    ("IQ2_S 1024 experts, T=3", dict(n_embd=512, n_ff=512, n_ff_shared=512, n_expert=1024, top_k=8, w_type=22,
                                     sh_type=22), 3, 45, True),
    ("IQ2_S n_ff=2048", dict(n_embd=512, n_ff=2048, n_ff_shared=2048, n_expert=16, top_k=4, w_type=22, sh_type=22),
     6, 46, True),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_forward_iq2_s_parity(torch, case):
    name, gkw, T, seed, add_shared = CASES[case]
    say(f"case: forward {name} T={T}")
    g = O.Geom(**gkw)
    w_host = O.make_weights(g, seed)
    w_dev = S.synth_layer(S.Geom(**vars(g)), seed)
    x = O.gen_normal(seed, 100, T * g.n_embd).reshape(T, g.n_embd)
    ml = S.MoELayer(S.Geom(**vars(g)), w_dev, max_tokens=T)
    yg = torch.full((T * g.n_embd + GUARD,), 7.0, dtype=torch.float32, device="cuda")
    yv = yg[:T * g.n_embd].view(T, g.n_embd)
    _, tr = ml.forward(dev(torch, x), y=yv, add_shared=add_shared, trace=True)
    got = host(torch, yg)
    assert (got[T * g.n_embd:] == 7.0).all(), "guard words past y were written"
    y = got[:T * g.n_embd].reshape(T, g.n_embd)
    want, wtr = O.moe_decode_dev(g, w_host, x, add_shared=add_shared, trace=True, n_threads=16)
    for k in ("logits", "ids", "weights", "counts", "offsets", "perm", "slot"):
        assert np.array_equal(bits(host(torch, tr[k])), bits(wtr[k])), k
    assert np.array_equal(bits(y), bits(want)), f"max rel {O.rel_l1_rows(y, want).max()}"
    # north_star's 1e-3 per row against the reference-order chain, or the reference's stage-wise check for a row
    # beyond it
    def stages():
        yy, st = ml.forward(dev(torch, x), add_shared=add_shared, trace=True, stages=True)
        return {k: host(torch, v) for k, v in st.items()}, host(torch, yy)
    SW.reference_order_gate(g, w_host, x, y, add_shared, stages, say, n_threads=16)
    if name.startswith("config 4"):
        D = int((host(torch, tr["counts"]) > 0).sum())
        say(f"  distinct experts touched: {D}")
        assert 300 < D < 420  # uniform routing of 64 x 10 pairs over 512 experts: E[D] ~ 367


def test_iq2_s_refusals(torch):
    say("case: IQ2_S refusals")
    ok = S.Geom(n_embd=512, n_ff=512, n_ff_shared=512, n_expert=16, top_k=4, w_type=22, sh_type=22)
    assert S.workspace_bytes(ok, 8) > 0
    # (a Q2_0 shared expert beside IQ2_S experts is a native shared expert now: tests/test_gpu_native.py)
    for bad in (dict(n_embd=768), dict(n_ff=256), dict(n_embd=4096), dict(n_ff_shared=1024)):
        kw = dict(vars(ok)); kw.update(bad)
        with pytest.raises(S.SmoeError):
            S.workspace_bytes(S.Geom(**kw), 8)
    w = S.synth_layer(ok, 3)
    ml = S.MoELayer(ok, w, max_tokens=8)
    with pytest.raises(S.SmoeError):
        ml.forward(torch.zeros((4, 512), device="cuda"), path=S.PATH_MFMA)
    # the automatic path stays on the IQ2_S GEMV kernels at prefill sizes
    ml2 = S.MoELayer(ok, w, max_tokens=130)
    x = O.gen_normal(9, 100, 130 * 512).reshape(130, 512)
    y = host(torch, ml2.forward(dev(torch, x)))
    assert np.array_equal(bits(y), bits(O.moe_decode_dev(O.Geom(**vars(ok)), O.make_weights(O.Geom(**vars(ok)), 3), x,
                                                           n_threads=16)))


@pytest.mark.parametrize("d_type,n_ff,n_tok", [(42, 512, 3), (22, 512, 2), (42, 1024, 1)])
def test_expert_blob_bitwise(torch, d_type, n_ff, n_tok):
    """smoe_expert (the reference's iq_expert): gate and up IQ2_S rows, SwiGLU to q8_1, down rows of d_type, on
    one [gate | up | down] blob; bitwise against the oracle's stage functions composed the same way
    (metal/src/iq.mm:182-199)."""
    say(f"case: expert blob d_type={d_type} n_ff={n_ff} n_tok={n_tok}")
    n_embd = 2048
    g = O.gen_iq2_s(61, 1, n_ff * n_embd // 256)
    u = O.gen_iq2_s(61, 2, n_ff * n_embd // 256)
    d = O.gen_q2_0(61, 3, n_embd * n_ff // 64) if d_type == 42 else O.gen_iq2_s(61, 3, n_embd * n_ff // 256)
    blob = np.concatenate([g.view(np.uint8).ravel(), u.view(np.uint8).ravel(), d.view(np.uint8).ravel()])
    assert blob.size == S.lib().smoe_expert_bytes(22, d_type, n_embd, n_ff)
    xq = O.quant_q8_1(O.gen_normal(61, 4, n_tok * n_embd))
    y = host(torch, S.expert(dev(torch, blob), dev(torch, xq), 22, d_type, n_embd, n_ff, n_tok))
    xb = n_embd // 32 * 36
    gate = np.concatenate([O.iq2_s_gemv_dev(g, xq[c * xb:(c + 1) * xb], n_embd, n_ff) for c in range(n_tok)])
    up = np.concatenate([O.iq2_s_gemv_dev(u, xq[c * xb:(c + 1) * xb], n_embd, n_ff) for c in range(n_tok)])
    hq = O.swiglu_q8(gate, up)
    hb = n_ff // 32 * 36
    for c in range(n_tok):
        want = O.gemv_dev(d_type, d, hq[c * hb:(c + 1) * hb], n_ff, n_embd)
        assert np.array_equal(bits(y[c]), bits(want)), c
