"""GPU parity of the other native GGUF types (smoe_native.hip) through the C ABI, against the oracle
(oracle/smoe_native.c, pinned by tests/test_oracle_native.py).

- smoe_mmvq for Q8_0, Q4_0, Q5_0, IQ4_NL, IQ4_XS, Q3_K, Q4_K, Q5_K, Q6_K: bitwise against or_native_gemv (the
  reference's 32-lane MMVQ order) over ragged row counts and column counts; refusals launch nothing.
- A layer whose shared expert is stored in its own types (gate, up and down each its own, as real layers:
  include/strata/kernels/shared_expert.hpp:54-58): decode bitwise against or_moe_decode_dev on every decode launch
  shape (the fused small batch, its unfused kernels, many tokens), the shared expert's output rows bitwise; the
  prefill path within 1e-3 per row of or_moe_prefill routed from the device's logits (tests/prefill_check.py)."""
import sys

import numpy as np
import pytest

import oracle as O
import prefill_check as PC
import stagewise as SW
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


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(torch, t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


TYPES = sorted(O.NATIVE)


@pytest.mark.parametrize("t", TYPES)
def test_mmvq_native_bitwise(torch, t):
    qk = O.NATIVE[t][0]
    shapes = [(qk, 1, 1), (4 * qk if qk == 256 else 640, 7, 3), (2048, 64, 1), (2304 if qk == 256 else 2080, 517, 2),
              (512, 33, 70)]
    for n_in, n_out, n_col in shapes:
        say(f"case: mmvq type {t} n_in={n_in} n_out={n_out} n_col={n_col}")
        w = O.gen_native_blocks(t, 7, n_in + n_out, n_in * n_out)
        x = O.gen_normal(t, n_in, n_col * n_in).reshape(n_col, n_in)
        xq = O.quant_q8_1(x)
        y = S.mmvq(t, dev(torch, w), dev(torch, xq), n_in, n_out, n_col)
        want = O.native_gemv(t, w, xq, n_in, n_out, n_col)
        assert np.array_equal(bits(host(torch, y)), bits(want)), (n_in, n_out, n_col)


def test_mmvq_native_refusals(torch):
    say("case: mmvq native refusals")
    w = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    xq = torch.zeros(36 * 8, dtype=torch.uint8, device="cuda")
    y = torch.full((4,), 7.0, dtype=torch.float32, device="cuda")
    L = S.lib()
    # IQ4_XS rows are whole 256-value blocks
    assert L.smoe_mmvq(O.IQ4_XS, w.data_ptr(), 0, xq.data_ptr(), 128, 1, 1, y.data_ptr(), S._stream()) == -1
    # Q4_0 rows of 33 values
    assert L.smoe_mmvq(O.Q4_0, w.data_ptr(), 0, xq.data_ptr(), 33, 1, 1, y.data_ptr(), S._stream()) == -1
    # an unknown type (F16 = 1)
    assert L.smoe_mmvq(1, w.data_ptr(), 0, xq.data_ptr(), 32, 1, 1, y.data_ptr(), S._stream()) == -3
    # misaligned weights
    assert L.smoe_mmvq(O.Q8_0, w.data_ptr(), 2, xq.data_ptr(), 32, 1, 1, y.data_ptr(), S._stream()) == -5
    assert (host(torch, y) == 7.0).all(), "a refused call wrote its output"


def native_layer(torch, g, seed):
    """Host weights from the oracle's generators (native shared blocks from numpy) and the same bytes on the device:
    the routed experts, router and shared gate from the device generator (bitwise the host's), the native shared
    projections uploaded."""
    w_host = O.make_weights(g, seed)
    base = S.Geom(**{k: v for k, v in vars(g).items() if k not in ("sh_gate_type", "sh_up_type", "sh_down_type")})
    base.sh_type = g.w_type
    w_dev = S.synth_layer(base, seed)
    for n in ("gate_sh", "up_sh", "down_sh"):
        w_dev[n] = dev(torch, getattr(w_host, n))
    return w_host, w_dev


CASES = [
    # name, geometry, T, seed, add_shared
    ("Q3_K gate/up, IQ4_NL down, b=1", dict(n_expert=64, top_k=8, sh_type=O.Q3_K, sh_down_type=O.IQ4_NL), 1, 61, True),
    ("IQ4_XS gate/up, Q4_0 down, fused small batch T=3",
     dict(n_expert=64, top_k=8, sh_type=O.IQ4_XS, sh_down_type=O.Q4_0), 3, 62, True),
    ("Q6_K gate, Q4_K up, Q8_0 down, b=16",
     dict(n_expert=64, sh_type=O.Q6_K, sh_up_type=O.Q4_K, sh_down_type=O.Q8_0), 16, 63, True),
    ("Q5_K gate/up, Q2_0 down (the Q2_0 GEMV then the gate scale)",
     dict(n_expert=64, sh_type=O.Q5_K, sh_down_type=O.Q2_0), 5, 64, True),
    ("Q2_0 gate/up, Q5_0 down, shared not added", dict(n_expert=64, sh_type=O.Q2_0, sh_down_type=O.Q5_0), 2, 65, False),
    ("IQ2_S routed, Q8_0 shared", dict(n_embd=512, n_ff=512, n_ff_shared=512, n_expert=16, top_k=4, w_type=22,
                                      sh_type=O.Q8_0), 6, 66, True),
    ("IQ2_S routed, Q2_0 shared (the Q2_0 GEMV chain)", dict(n_embd=512, n_ff=512, n_ff_shared=512, n_expert=16,
                                                            top_k=4, w_type=22, sh_type=O.Q2_0), 3, 70, True),
    ("full geometry, Q3_K gate/up, IQ4_NL down, b=1", dict(sh_type=O.Q3_K, sh_down_type=O.IQ4_NL), 1, 67, True),
    ("reference width FF 640: IQ4_NL down", dict(n_embd=2560, n_ff=640, n_ff_shared=640, n_expert=32, top_k=4,
                                                 sh_type=O.Q2_0, sh_down_type=O.IQ4_NL), 4, 68, True),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_forward_native_shared_decode(torch, case):
    name, gkw, T, seed, add_shared = CASES[case]
    say(f"case: native shared {name} T={T}")
    g = O.Geom(**gkw)
    w_host, w_dev = native_layer(torch, g, seed)
    x = O.gen_normal(seed, 100, T * g.n_embd).reshape(T, g.n_embd)
    ml = S.MoELayer(S.Geom(**vars(g)), w_dev, max_tokens=T)
    y, tr = ml.forward(dev(torch, x), add_shared=add_shared, trace=True)
    want, wtr = O.moe_decode_dev(g, w_host, x, add_shared=add_shared, trace=True, n_threads=8)
    for k in ("ids", "weights", "perm", "slot", "sgate"):
        assert np.array_equal(bits(host(torch, tr[k])), bits(wtr[k])), k
    assert np.array_equal(bits(host(torch, y)), bits(want)), f"max rel {O.rel_l1_rows(host(torch, y), want).max()}"
    # the traced call (unfused kernels) gives the same bits and the shared expert's rows
    y2, tr2 = ml.forward(dev(torch, x), add_shared=add_shared, trace=True, stages=True)
    assert np.array_equal(bits(host(torch, y2)), bits(want))
    assert np.array_equal(bits(host(torch, tr2["shared"])), bits(wtr["shared"]))
    # the reference-order chain: 1e-3 per row, or the reference's stage-wise check for a row beyond it
    htr2 = {k: host(torch, v) for k, v in tr2.items()}
    rep = SW.stagewise(g, w_host, x, htr2, host(torch, y2), add_shared)
    say(f"  stage-wise: {rep.summary()}")
    assert rep.ok(), rep.summary()
    SW.reference_order_gate(g, w_host, x, host(torch, y), add_shared, lambda: (htr2, host(torch, y2)), say)


def test_forward_native_shared_prefill(torch):
    g = O.Geom(n_expert=64, top_k=8, sh_type=O.Q3_K, sh_down_type=O.IQ4_NL)
    T, seed = 160, 69
    say(f"case: native shared prefill T={T}")
    w_host, w_dev = native_layer(torch, g, seed)
    x = O.gen_normal(seed, 100, T * g.n_embd).reshape(T, g.n_embd)
    ml = S.MoELayer(S.Geom(**vars(g)), w_dev, max_tokens=T)
    y, tr = ml.forward(dev(torch, x), trace=True, path=S.PATH_MFMA)
    htr = {k: host(torch, v) for k, v in tr.items()}
    PC.router_stagewise(g, w_host, x, htr)  # the router on the matrix cores; the routing of its logits exact
    want = PC.prefill_want(g, w_host, x, htr, n_threads=8)
    assert O.rel_l1_rows(host(torch, y), want).max() <= 1e-3
