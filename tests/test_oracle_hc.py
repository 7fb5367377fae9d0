"""CPU tests of the test oracle's hyper-connection ends (gr_read / gr_write of FfnExec::run), pinned the way the
reference pins its own (metal/src/gr_parity.cpp): an independent float64 evaluation of the read (numpy, here) that
both oracle orders must meet within 1e-4 rel_l1 for mixed and inject; traps showing that each plausible slip (the norm
over the whole stack, /hc outside the silu, silu and sigmoid swapped, a sum instead of the mean, unrounded
activations) moves the result by more than that; the reference's scalar closed form; and the write's closed forms
(a zero injection is a plain residual add, 2 sigmoid and not sigmoid, every stream gets the same block output)."""
import numpy as np
import pytest

import oracle as O

TOL = 1e-4


def bf16(x):
    return O.f32_from_bf16(O.bf16_from_f32(np.asarray(x, np.float32)))


def read_f64(R, n, w, per_stream=True, inside=True, gate_sigmoid=True, mean=True, round_act=True):
    """gr_read in float64 with the reference test's switches (metal/src/gr_parity.cpp:95-168)."""
    hc, hc_lr = w.hc, w.hc_lr
    hd = hc * n
    R = np.asarray(R, np.float64).reshape(-1, hd)
    down = O.f32_from_bf16(w.down).astype(np.float64).reshape(hc_lr, hd)
    up = O.f32_from_bf16(w.up).astype(np.float64).reshape(hd, hc_lr)
    inj = O.f32_from_bf16(w.inject).astype(np.float64).reshape(hc, hd)
    norm = w.norm.astype(np.float64)
    mixed, inject = [], []
    sig = lambda z: 1.0 / (1.0 + np.exp(-z))
    silu = lambda z: z * sig(z)
    for r in R:
        if per_stream:
            ms = (r.reshape(hc, n) ** 2).mean(axis=1)
            rs = np.repeat(1.0 / np.sqrt(ms + w.eps), n)
        else:
            rs = np.full(hd, 1.0 / np.sqrt((r ** 2).mean() + w.eps))
        xn = r * rs * norm
        act = bf16(xn).astype(np.float64) if round_act else xn
        p = down @ act
        lo = (silu(p / hc) if inside else silu(p) / hc) if gate_sigmoid else (sig(p / hc) if inside else sig(p) / hc)
        lq = bf16(lo).astype(np.float64) if round_act else lo
        gate = up @ lq
        s = sig(gate) if gate_sigmoid else silu(gate)
        m = (xn * s).reshape(hc, n).sum(axis=0)
        mixed.append(m / hc if mean else m)
        inject.append(inj @ act)
    return np.array(mixed), np.array(inject)


def rel_l1(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return np.abs(a - b).sum() / max(np.abs(b).sum(), 1e-30)


def fixture(n, hc, hc_lr, seed, T=2):
    w = O.make_hc(n, hc, hc_lr, seed)
    R = O.gen_normal(seed, 41, T * hc * n).reshape(T, hc, n)
    R = R * (4.0 ** np.arange(hc, dtype=np.float32))[None, :, None]  # streams of very different scales
    return w, R.astype(np.float32)


@pytest.mark.parametrize("n,hc,hc_lr", [(256, 4, 32), (2048, 4, 320), (512, 2, 64)])
def test_read_orders_meet_the_f64_evaluation(n, hc, hc_lr):
    w, R = fixture(n, hc, hc_lr, 1234 + n)
    want_m, want_i = read_f64(R, n, w)
    for fn in (O.hc_read_dev, O.hc_read_ref):
        m, i = fn(R, n, w)
        assert rel_l1(m, want_m) <= TOL and rel_l1(i, want_i) <= TOL, fn.__name__
    # the f32-activation contract of the reference (fp32_act) against its own f64 evaluation
    m32, i32 = O.hc_read_ref(R, n, w, round_act=False)
    wm, wi = read_f64(R, n, w, round_act=False)
    assert rel_l1(m32, wm) <= TOL and rel_l1(i32, wi) <= TOL


def test_read_traps_are_observable():
    n, hc, hc_lr = 256, 4, 32
    w, R = fixture(n, hc, hc_lr, 77)
    right, _ = read_f64(R, n, w)
    got, _ = O.hc_read_dev(R, n, w)
    assert rel_l1(got, right) <= TOL
    traps = [(dict(per_stream=False), 0.05), (dict(inside=False), 0.05), (dict(gate_sigmoid=False), 0.05),
             (dict(mean=False), 0.5), (dict(round_act=False), TOL)]
    for kw, floor in traps:
        wrong, _ = read_f64(R, n, w, **kw)
        assert rel_l1(wrong, right) > floor, kw
        assert rel_l1(got, wrong) > floor, kw  # the oracle is not the slipped formula


@pytest.mark.parametrize("gamma", [1.0, 1.00390625])
def test_read_scalar_closed_form(gamma):
    """The reference's scalar case (metal/src/gr_parity.cpp:381-420), padded to whole 8-value chunks: unit streams,
    norm gamma, one non-zero down weight 0.5, up weights 1.5 on lq_0, inject weight 2."""
    n, hc, hc_lr = 8, 1, 8
    w = O.HcWeights(hc, hc_lr, 0.0, np.full(n, gamma, np.float32), np.zeros(hc_lr * n, np.uint16),
                    np.zeros(n * hc_lr, np.uint16), np.zeros(n, np.uint16))
    w.down[0] = O.bf16_from_f32(np.float32([0.5]))[0]
    w.up.reshape(n, hc_lr)[:, 0] = O.bf16_from_f32(np.float32(1.5))
    w.inject[0] = O.bf16_from_f32(np.float32([2.0]))[0]
    R = np.ones((1, hc, n), np.float32)
    act = float(bf16([gamma])[0])
    lo = (act * 0.5) / (1.0 + np.exp(-(act * 0.5)))
    want_m = gamma / (1.0 + np.exp(-float(bf16([lo])[0]) * 1.5))
    for fn in (O.hc_read_dev, O.hc_read_ref):
        m, i = fn(R, n, w)
        assert np.all(np.abs(m - want_m) <= 2e-7) and np.all(m == m[0, 0]), fn.__name__
        assert i[0, 0] == np.float32(act * 2.0)


def test_write_closed_forms():
    n, hc, T = 256, 4, 3
    R = O.gen_normal(5, 50, T * hc * n).reshape(T, hc, n)
    y = O.gen_normal(5, 51, T * n).reshape(T, n)
    out0 = O.hc_write_dev(R, y, np.zeros((T, hc), np.float32), n, hc)
    assert np.array_equal(out0, (R + y[:, None, :]).astype(np.float32))  # 2 sigmoid(0) = 1 exactly
    inj = (O.gen_normal(5, 52, T * hc) * 3.0).reshape(T, hc)
    out = O.hc_write_dev(R, y, inj, n, hc).astype(np.float64)
    s2 = 2.0 / (1.0 + np.exp(-inj.astype(np.float64) / hc))
    term = y.astype(np.float64)[:, None, :] * s2[:, :, None]
    want = R.astype(np.float64) + term
    assert (np.abs(out - want) / (np.abs(R) + np.abs(term))).max() < 1e-6
    half = R.astype(np.float64) + term / 2.0  # the 1 * sigmoid slip
    assert rel_l1(out - R, half - R) > 0.05
