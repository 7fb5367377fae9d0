"""The oracle's restatement of the other native GGUF types (oracle/smoe_native.c), pinned without a GPU.

- The blocks' values equal the reference's own dequantisers bit for bit (include/strata/artifact/dequant.hpp:81-280):
  live through oracle/_ref where the reference tree is present, and against the committed vectors in
  tests/golden/native_ref.npz (edge scales included) everywhere.
- The q8_1 integer partials in the reference's 32-lane order (metal/shaders/iq.metal:224-513, its host restatements
  metal/src/pack_parity.cpp:2785-3475) agree with an independent evaluation: the dequantised weights times the
  dequantised q8_1 values summed in double, within 1e-6 of each row's absolute sum (f32 rounding of the partials).
- The check sees a one-code mistake: changing a single code bit of a block moves the double evaluation by more than
  ten times that tolerance for most bits, so a wrong index, sign or bias in a partial cannot hide in it.
- Closed forms: zero activations give zero; zero block scales give zero.
"""
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TYPES = sorted(O.NATIVE)
TOL = 1e-6


def q8_values(xq: np.ndarray, n_col: int, n: int) -> np.ndarray:
    b = xq.reshape(-1, 36)
    d = O.f32_from_f16(b[:, :2].copy().view(np.uint16).ravel()).astype(np.float64)
    q = b[:, 4:].view(np.int8).astype(np.float64)
    return (q * d[:, None]).reshape(n_col, n)


@pytest.mark.parametrize("t", TYPES)
def test_native_dequant_golden_vectors(t):
    f = np.load(os.path.join(GOLD, "native_ref.npz"))
    b, want = f[f"blocks_{t}"], f[f"values_{t}"]
    got = O.native_dequant(t, b, want.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
def test_native_dequant_matches_reference_live(t):
    if O.ref() is None:
        pytest.skip("oracle/_ref absent (no /root/reference here): the committed vectors pin the dequantisers")
    qk = O.NATIVE[t][0]
    for seed in range(3):
        n = qk * 97
        b = O.gen_native_blocks(t, seed, 11, n, sigma=0.5 if seed == 2 else 0.02)
        assert np.array_equal(O.native_dequant(t, b, n).view(np.uint32), O.ref_dequantize(t, b, n).view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("n_in", [256, 512, 2304])
def test_native_gemv_matches_double(t, n_in):
    rng = np.random.default_rng(n_in + t)
    n_out, n_col = 19, 3
    w = O.gen_native_blocks(t, 5, n_in, n_in * n_out)
    x = (rng.normal(size=(n_col, n_in)) * np.exp(rng.normal(size=(n_col, 1)))).astype(np.float32)
    xq = O.quant_q8_1(x)
    y = O.native_gemv(t, w, xq, n_in, n_out, n_col)
    yd = O.native_gemv(t, w, xq, n_in, n_out, n_col, double=True)
    W = O.native_dequant(t, w, n_in * n_out).reshape(n_out, n_in).astype(np.float64)
    absum = (np.abs(W) @ np.abs(q8_values(xq, n_col, n_in)).T).T
    assert np.all(np.abs(y.astype(np.float64) - yd) <= TOL * absum + 1e-30)
    # the independent evaluation itself: numpy's double product of the same values
    assert np.allclose(yd, (W @ q8_values(xq, n_col, n_in).T).T.astype(np.float32), rtol=1e-6, atol=1e-12)


@pytest.mark.parametrize("t", TYPES)
def test_native_one_code_mistake_is_visible(t):
    qk, nb, fields, _ = O.NATIVE[t]
    n_in = 512
    rng = np.random.default_rng(t)
    w = O.gen_native_blocks(t, 9, 3, n_in)
    xq = O.quant_q8_1(rng.normal(size=n_in).astype(np.float32))
    y = float(O.native_gemv(t, w, xq, n_in, 1, 1)[0, 0])
    a = q8_values(xq, 1, n_in)[0]
    absum = float(np.abs(O.native_dequant(t, w, n_in)).astype(np.float64) @ np.abs(a))
    kb = int(np.argmax(np.abs(O.native_dequant(t, w, n_in)).reshape(-1, qk).max(axis=1)))  # the strongest block
    moved = 0
    for byte in range(nb):  # every non-scale byte of that block, one bit at a time
        if any(f <= byte < f + 2 for f in fields):
            continue
        w2 = w.copy()
        w2[kb * nb + byte] ^= 0x01
        y2 = float(O.native_gemv(t, w2, xq, n_in, 1, 1, double=True)[0, 0])
        if abs(y2 - y) > 10 * TOL * absum:  # ten times the tolerance of test_native_gemv_matches_double
            moved += 1
    assert moved >= (nb - 2 * len(fields)) // 2, f"only {moved} single-bit changes were visible"


@pytest.mark.parametrize("t", TYPES)
def test_native_closed_forms(t):
    qk, nb, fields, _ = O.NATIVE[t]
    n_in, n_out = 256, 4
    w = O.gen_native_blocks(t, 2, 2, n_in * n_out)
    zq = O.quant_q8_1(np.zeros(n_in, np.float32))
    assert np.all(O.native_gemv(t, w, zq, n_in, n_out, 1) == 0.0)
    w0 = w.reshape(-1, nb).copy()
    for f in fields:
        w0[:, f:f + 2] = 0
    xq = O.quant_q8_1(np.random.default_rng(1).normal(size=n_in).astype(np.float32))
    assert np.all(O.native_gemv(t, w0.ravel(), xq, n_in, n_out, 1) == 0.0)


def test_native_partition_matches_reference_order():
    """Q4_0 by hand: two partials per 32-value block (iqs 0, 2), lane k & 31 adds them in order, butterfly 16..1."""
    t, n_in = O.Q4_0, 1024
    w = O.gen_native_blocks(t, 3, 3, n_in)
    xq = O.quant_q8_1(np.random.default_rng(3).normal(size=n_in).astype(np.float32))
    lib = O.lib()
    lane = np.zeros(32, np.float32)
    for k in range(n_in // 32 * 2):
        kb = k // 2
        blk = w[kb * 18:(kb + 1) * 18].copy()
        x0 = xq[kb * 36:(kb + 1) * 36].copy()
        p = np.float32(lib.or_native_part(t, blk.ctypes.data, x0.ctypes.data, 2 * (k % 2)))
        lane[k & 31] = np.float32(lane[k & 31] + p)
    for o in (16, 8, 4, 2, 1):
        lane = (lane + lane[np.arange(32) ^ o]).astype(np.float32)
    assert lane[0].view(np.uint32) == O.native_gemv(t, w, xq, n_in, 1, 1)[0, 0].view(np.uint32)
