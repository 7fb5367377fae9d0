"""CPU tests of the oracle (oracle/): pinned against the reference's own compiled codecs (oracle/_ref or the
committed vectors in tests/golden/codecs_ref.npz), libm / numpy, closed forms, brute force and the reference
tests' known answers and traps (metal/src/{router,moe_combine,iq}_parity.cpp)."""
import hashlib
import math
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def codecs():
    return np.load(os.path.join(GOLD, "codecs_ref.npz"))


# ------------------------------------------------------------------------------------------------ A1 codecs

def test_f16_encode_matches_reference_vectors(codecs):
    x = codecs["x"]
    assert np.array_equal(O.f16_from_f32(x), codecs["f16"])


def test_bf16_encode_matches_reference_vectors(codecs):
    assert np.array_equal(O.bf16_from_f32(codecs["x"]), codecs["bf16"])


def test_f16_decode_exhaustive_matches_reference(codecs):
    allh = np.arange(65536, dtype=np.uint16)
    assert sha(O.f32_from_f16(allh)) == str(codecs["f16_decode_sha"])


def test_f16_against_numpy_float16():
    # numpy's float16 is the oracle the reference used for its converter (include/strata/kernels/f16_bits.hpp:7-10)
    rng = np.random.default_rng(5)
    x = rng.integers(0, 2 ** 32, 500_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[np.isfinite(x)]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f16_from_f32(x), want)
    allh = np.arange(65536, dtype=np.uint16)
    fin = np.isfinite(allh.view(np.float16))
    assert np.array_equal(O.f32_from_f16(allh)[fin], allh.view(np.float16)[fin].astype(np.float32))


def test_bf16_tie_rounds_to_even_and_nan_is_quiet():
    # 1 + 2^-8 is an exact bf16 tie between 1 and 1 + 2^-7: the even neighbour is 1.0 (0x3F80)
    assert O.bf16_from_f32(np.array([1.0 + 2 ** -8], np.float32))[0] == 0x3F80
    assert O.bf16_from_f32(np.array([1.0 + 3 * 2 ** -8], np.float32))[0] == 0x3F82
    nan = np.array([0x7FFFFFFF], np.uint32).view(np.float32)
    assert O.bf16_from_f32(nan)[0] & 0x7FC0 == 0x7FC0


def test_oracle_codecs_against_live_reference_build():
    R = O.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (no /root/reference here); the committed vectors cover it")
    rng = np.random.default_rng(11)
    x = rng.integers(0, 2 ** 32, 1_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    a = np.empty(x.size, np.uint16)
    R.ref_f16_from_f32_n(x.ctypes.data, x.size, a.ctypes.data)
    assert np.array_equal(O.f16_from_f32(x), a)
    R.ref_bf16_from_f32_n(x.ctypes.data, x.size, a.ctypes.data)
    assert np.array_equal(O.bf16_from_f32(x), a)


# ------------------------------------------------------------------------------------------------ elementary functions

def test_expf_within_one_ulp_of_correctly_rounded():
    L = O.lib()
    xs = np.concatenate([np.linspace(-87, 88.7, 40001), np.linspace(-1, 1, 20001)]).astype(np.float32)
    got = np.array([L.or_expf(float(v)) for v in xs], np.float32)
    want = np.exp(xs.astype(np.float64)).astype(np.float32)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1
    assert L.or_expf(-100.0) == 0.0 and math.isinf(L.or_expf(100.0)) and L.or_expf(0.0) == 1.0


def test_logf_and_cos2pi_accuracy():
    L = O.lib()
    us = np.concatenate([np.geomspace(5.96e-8, 1.0, 20001), np.linspace(0.5, 1.0, 5001)]).astype(np.float32)
    lg = np.array([L.or_logf(float(v)) for v in us], np.float64)
    ln = np.log(us.astype(np.float64))
    assert np.max(np.abs(lg - ln) / np.maximum(1.0, np.abs(ln))) < 1.2e-7   # about 2 ulp
    cs = np.array([L.or_cos2pi(float(v)) for v in us], np.float64)
    assert np.max(np.abs(cs - np.cos(2 * np.pi * us.astype(np.float64)))) < 2e-7
    assert L.or_cos2pi(0.0) == 1.0 and L.or_cos2pi(0.5) == -1.0


def test_generators_are_normal_and_counter_based():
    n = O.gen_normal(7, 1, 400_000)
    assert abs(n.mean()) < 0.01 and abs(n.std() - 1) < 0.01
    assert abs(((n - n.mean()) ** 4).mean() / n.var() ** 2 - 3.0) < 0.05
    # counter based: a slice equals the same indices of a longer run
    assert np.array_equal(O.gen_normal(7, 1, 1000), n[:1000])
    assert not np.array_equal(O.gen_normal(7, 2, 1000), n[:1000])


# ------------------------------------------------------------------------------------------------ A2 Q2_0

def test_q2_0_dequant_matches_reference_vectors(codecs):
    got = O.dequant_q2_0(codecs["q2_blocks"])
    assert np.array_equal(got.view(np.uint32), codecs["q2_dequant"].view(np.uint32))


def test_q2_0_structural_invariant():
    # every value is one of {-d, 0, d, 2d} of its own block (include/strata/artifact/dequant.hpp:15-18)
    b = O.gen_q2_0(3, 3, 500)
    v = O.dequant_q2_0(b).reshape(500, 64)
    d = O.f32_from_f16(b.reshape(500, 18)[:, :2].copy().view(np.uint16).ravel())
    ok = np.zeros_like(v, bool)
    for s in (-1, 0, 1, 2):
        ok |= v == (np.float32(s) * d[:, None])
    assert ok.all()
    # the symbol distribution of uniform code bytes is uniform over {-1, 0, 1, 2}
    counts = np.array([(v == s * d[:, None]).sum() for s in (-1, 1, 2)])
    assert np.all(np.abs(counts / v.size - 0.25) < 0.01)


# ------------------------------------------------------------------------------------------------ A3 q8_1

def _q8_fields(blk):
    d = O.f32_from_f16(blk[0:2].copy().view(np.uint16))[0]
    s = O.f32_from_f16(blk[2:4].copy().view(np.uint16))[0]
    q = blk[4:36].view(np.int8)
    return d, s, q


def test_q8_1_known_answers():
    # metal/src/iq_parity.cpp:456-464: a huge value clamps d to 65504 and q to 127
    x = O.gen_normal(1, 1, 128)
    x[3] = 1e10
    x[40] = -8e6
    y = O.quant_q8_1(x)
    d0, s0, q0 = _q8_fields(y[0:36])
    assert d0 == 65504.0 and q0[3] == 127 and s0 == 65504.0
    assert np.all(q0[np.arange(32) != 3] == 0)
    d1, s1, q1 = _q8_fields(y[36:72])
    assert q1[8] == -127 and d1 == np.float32(O.f32_from_f16(O.f16_from_f32(np.array([8e6 / 127], np.float32))))[0]
    # an all-zero block: d = 0, q = 0
    z = O.quant_q8_1(np.zeros(32, np.float32))
    assert not z.any()


def test_q8_1_closed_form():
    x = O.gen_normal(2, 2, 32 * 200).reshape(200, 32)
    y = O.quant_q8_1(x).reshape(200, 36)
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(y[:, 0:2].copy().view(np.uint16).ravel(), O.f16_from_f32(d))
    q = np.clip(np.floor(np.abs(x / d[:, None]) + 0.5) * np.sign(x), -127, 127).astype(np.int8)
    assert np.array_equal(y[:, 4:].view(np.int8), q)


# ------------------------------------------------------------------------------------------------ A4 Q2_0 x q8_1

@pytest.mark.parametrize("n_in,n_out", [(128, 3), (2048, 40), (512, 64), (2560, 8), (640, 16)])
def test_q2_0_gemv_orders_against_brute_force(n_in, n_out):
    w = O.gen_q2_0(5, n_in, n_out * n_in // 64)
    xq = O.quant_q8_1(O.gen_normal(5, n_out, n_in))
    exact = O.q2_0_gemv_exact(w, xq, n_in, n_out)
    dev = O.q2_0_gemv_dev(w, xq, n_in, n_out)
    ref = O.q2_0_gemv_ref(w, xq, n_in, n_out)
    assert O.rel_l1_rows(dev[None], exact[None])[0] < 1e-6
    assert O.rel_l1_rows(ref[None], exact[None])[0] < 1e-6
    assert O.rel_l1_rows(dev[None], ref[None])[0] <= 1e-5


def test_q2_0_trap_forgetting_minus_one_is_observable():
    # metal/src/iq_parity.cpp:510-522: a code that forgets the -1 must land more than 5% away
    n_in, n_out = 256, 4
    w = O.gen_q2_0(8, 8, n_out * n_in // 64)
    xq = O.quant_q8_1(O.gen_normal(8, 9, n_in) + 0.3)
    good = O.q2_0_gemv_ref(w, xq, n_in, n_out)
    bad = O.q2_0_gemv_no_minus_one(w, xq, n_in, n_out)
    assert O.rel_l1_rows(bad[None], good[None])[0] > 0.05


def test_q2_0_gemv_brute_force_tiny():
    # one block, hand decoded: sum over 64 of (code - 1) * q, scaled per half block
    w = O.gen_q2_0(9, 9, 1)
    xq = O.quant_q8_1(O.gen_normal(9, 10, 64))
    codes = np.array([(w[2 + j // 4] >> (2 * (j % 4))) & 3 for j in range(64)], np.int64)
    q = np.concatenate([xq[4:36].view(np.int8), xq[40:72].view(np.int8)]).astype(np.int64)
    dw = float(O.f32_from_f16(w[0:2].copy().view(np.uint16))[0])
    dx = [float(O.f32_from_f16(xq[36 * h:36 * h + 2].copy().view(np.uint16))[0]) for h in (0, 1)]
    want = sum(dw * dx[h] * float(((codes[32 * h:32 * h + 32] - 1) * q[32 * h:32 * h + 32]).sum()) for h in (0, 1))
    assert abs(O.q2_0_gemv_exact(w, xq, 64, 1)[0] - want) <= 1e-12 * max(1.0, abs(want))


# ------------------------------------------------------------------------------------------------ A8 IQ2_S

def test_iq2s_grid_matches_reference(codecs):
    assert sha(O.iq2s_grid()) == str(codecs["iq2s_grid_sha"])
    assert sha(O.iq2s_grid()) == "e1aa1473412b0552c2174c30ef22ab4073f6a181b85a17056e8249bd2932fd88"


def test_iq2s_codebook_copies_identical():
    """The kernels compile their own copy of the codebook table; it is the oracle's pinned one, byte for byte."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    with open(os.path.join(root, "oracle", "iq2s_grid_codes.inc"), "rb") as f:
        pinned = f.read()
    with open(os.path.join(root, "stratametal_amd", "csrc", "iq2s_grid_codes.inc"), "rb") as f:
        kernels = f.read()
    assert kernels == pinned


def _iq2s_brute(w, xq, n_in, n_out):
    grid = O.iq2s_grid()
    rb = n_in // 256 * 82
    out = np.zeros(n_out)
    for r in range(n_out):
        row = w[r * rb:(r + 1) * rb]
        acc = 0.0
        for b in range(n_in // 256):
            blk = row[b * 82:(b + 1) * 82]
            d = float(O.f32_from_f16(blk[0:2].copy().view(np.uint16))[0])
            for ib in range(8):
                xb = xq[(8 * b + ib) * 36:(8 * b + ib + 1) * 36]
                dx = float(O.f32_from_f16(xb[0:2].copy().view(np.uint16))[0])
                q = xb[4:36].view(np.int8).astype(np.int64)
                sums = []
                for grp in range(4):
                    idx = int(blk[2 + 4 * ib + grp]) | (((int(blk[66 + ib]) >> (2 * grp)) & 3) << 8)
                    mags = [(int(grid[idx]) >> (8 * j)) & 0xFF for j in range(8)]
                    sb = int(blk[34 + 4 * ib + grp])
                    vals = [-m if (sb >> j) & 1 else m for j, m in enumerate(mags)]
                    sums.append(int(np.dot(vals, q[8 * grp:8 * grp + 8])))
                s0, s1 = sums[0] + sums[1], sums[2] + sums[3]
                ls0, ls1 = int(blk[74 + ib]) & 15, int(blk[74 + ib]) >> 4
                t = s0 * ls0 + s1 * ls1 + int((s0 + s1) / 2)   # C truncation toward zero
                sumi = int(t / 4)
                acc += d * dx * sumi
        out[r] = acc
    return out


def test_iq2_s_gemv_against_brute_force():
    n_in, n_out = 512, 6
    w = O.gen_iq2_s(6, 6, n_out * n_in // 256)
    xq = O.quant_q8_1(O.gen_normal(6, 7, n_in))
    want = _iq2s_brute(w, xq, n_in, n_out)
    dev = O.iq2_s_gemv_dev(w, xq, n_in, n_out)
    ref = O.iq2_s_gemv_ref(w, xq, n_in, n_out)
    assert O.rel_l1_rows(dev[None], want[None])[0] < 1e-6
    assert O.rel_l1_rows(ref[None], want[None])[0] < 1e-6


# ------------------------------------------------------------------------------------------------ A5 router

def test_router_known_answers():
    E, K, T = 512, 10, 64
    # all equal (ties): ids 0..9, weights 0.1 (metal/src/router_parity.cpp:138-139)
    ids, w = O.route_dev(np.full((T, E), 0.5, np.float32), K)
    assert (ids == np.arange(K)).all() and np.allclose(w, 0.1, atol=1e-7)
    # 12-way exact tie on experts 0..11 at 2.0 (router_parity.cpp:141-144)
    c = O.gen_normal(3, 3, T * E).reshape(T, E)
    c[:, :12] = 2.0
    c = np.minimum(c, 1.9)
    c[:, :12] = 2.0
    ids, w = O.route_dev(c, K)
    assert (ids == np.arange(K)).all()
    # dominant expert t % E at 20 (router_parity.cpp:146-148)
    d = np.zeros((T, E), np.float32)
    d[np.arange(T), np.arange(T) % E] = 20.0
    ids, _ = O.route_dev(d, K)
    assert (ids[:, 0] == np.arange(T) % E).all()
    # trap: "highest index on a tie" differs from the rule in more than half the ids (router_parity.cpp:160-171)
    assert (np.arange(E - 1, E - 1 - K, -1) != np.arange(K)).mean() > 0.5
    # the 2^-14 clamp is unreachable at k/E (router_parity.cpp:150-158)
    assert K / E > 6.103515625e-05


def test_router_margin_pinned():
    """The router-margin diagnostic (metal/src/forward.cpp:441-513): a closed form on geometric logits, the all-equal
    tie, a float64 evaluation on random logits, and the rule that the ranking is the routing's own."""
    E, K = 512, 10
    # logits -0.1 e: p_e proportional to exp(-0.1 e), the k-th and (k+1)-th are experts k-1 and k
    l = (-0.1 * np.arange(E)).astype(np.float32)[None]
    st, ids = O.router_margin_dev(l, K)
    ll = l[0].astype(np.float64)
    p = np.exp(ll - ll.max()) / np.exp(ll - ll.max()).sum()
    assert list(ids[0]) == [K - 1, K]
    assert abs(st[0, 0] - (p[K - 1] - p[K])) <= 1e-7 and abs(st[0, 2] - p[K - 1]) <= 1e-7
    assert st[0, 1] == np.float32(l[0, K - 1] - l[0, K])
    # all equal: ids k-1 and k (ties to the lower id), margin exactly 0, p = 1/E
    st, ids = O.router_margin_dev(np.full((3, E), 0.5, np.float32), K)
    assert (ids == [K - 1, K]).all() and (st[:, 0] == 0).all() and np.allclose(st[:, 2], 1.0 / E, rtol=1e-6)
    # random logits: ids are the routing's k-th pick and its (k+1)-th; the margin within 1e-7 of float64
    T = 64
    lr = (O.gen_normal(9, 9, T * E) * 0.9).reshape(T, E)
    st, ids = O.router_margin_dev(lr, K)
    ids11, _ = O.route_dev(lr, K + 1)
    assert (ids[:, 0] == ids11[:, K - 1]).all() and (ids[:, 1] == ids11[:, K]).all()
    l64 = lr.astype(np.float64)
    p64 = np.exp(l64 - l64.max(axis=1, keepdims=True))
    p64 /= p64.sum(axis=1, keepdims=True)
    rows = np.arange(T)
    m64 = p64[rows, ids[:, 0]] - p64[rows, ids[:, 1]]
    assert np.abs(st[:, 0] - m64).max() <= 1e-7
    assert np.array_equal(st[:, 1], (lr[rows, ids[:, 0]] - lr[rows, ids[:, 1]]).astype(np.float32))
    with pytest.raises(ValueError):
        O.router_margin_dev(lr[:, :10], 10)


@pytest.mark.parametrize("T,E,K", [(64, 512, 10), (4, 7, 3), (4, 1024, 10), (2, 64, 64)])
def test_route_device_order_matches_reference_routing(T, E, K):
    logits = O.gen_normal(2024, E + K, T * E).reshape(T, E)
    ids_d, w_d = O.route_dev(logits, K)
    ids_r, w_r = O.route_ref(logits, K)
    assert np.array_equal(ids_d, ids_r)
    assert np.max(np.abs(w_d - w_r) / np.abs(w_r)) <= 1e-5
    assert np.max(np.abs(w_d.sum(axis=1) - 1.0)) <= 1e-5
    # trap: renormalisation left out moves the weights far (router_parity.cpp:173-180)
    if K < E:
        p = np.exp(logits.astype(np.float64) - logits.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        raw = np.take_along_axis(p, ids_r.astype(np.int64), axis=1)
        assert np.abs(raw - w_r).sum() / np.abs(w_r).sum() > 0.05


def test_router_gemv_orders():
    H, E = 2048, 64
    xb = O.gen_bf16(1, 1, H, 1.0)
    W = O.gen_bf16(1, 2, E * H, 0.02)
    dev = O.bf16_gemv_dev(xb, W, H, E)
    dbl = O.bf16_gemv_double(xb, W, H, E)
    exact = (O.f32_from_bf16(W).reshape(E, H).astype(np.float64) @ O.f32_from_bf16(xb).astype(np.float64))
    assert O.rel_l1_rows(dev[None], exact[None])[0] < 1e-6
    assert O.rel_l1_rows(dev[None], dbl[None])[0] <= 1e-5


def test_f32_router_gemv_orders():
    """The f32 router (router_dtype 1, the literal configs[0]): the device order against an exact float64 product,
    the reference-style double sum, a brute-force restatement of the lane order on a small row, and the trap that
    rounding x or W to bf16 (the repo's contract) is observable."""
    H, E = 2048, 64
    x = O.gen_normal(1, 1, H, 1.0)
    W = O.gen_normal(1, 2, E * H, 0.02)
    dev = O.f32_gemv_dev(x, W, H, E)
    dbl = O.f32_gemv_double(x, W, H, E)
    exact = W.reshape(E, H).astype(np.float64) @ x.astype(np.float64)
    assert O.rel_l1_rows(dev[None], exact[None])[0] < 1e-6
    assert O.rel_l1_rows(dev[None], dbl[None])[0] <= 1e-5
    assert np.array_equal(dbl, exact.astype(np.float32))
    bf = O.bf16_gemv_dev(O.bf16_from_f32(x), O.bf16_from_f32(W), H, E)
    assert O.rel_l1_rows(bf[None], exact[None])[0] > 1e-3
    # the lane order by hand: lane l fuses the products of chunks l, l + 64, ... in element order, then the butterfly
    n = 512
    xs, ws = x[:n], W[:n]
    lanes = []
    for l in range(64):
        acc = np.float32(0.0)
        for c in range(l, n // 4, 64):
            for i in range(4):
                acc = np.float32(np.float64(xs[4 * c + i]) * np.float64(ws[4 * c + i]) + np.float64(acc))
        lanes.append(acc)
    lanes = np.array(lanes, np.float32)
    for o in (32, 16, 8, 4, 2, 1):
        lanes = (lanes + lanes[np.arange(64) ^ o]).astype(np.float32)
    assert O.f32_gemv_dev(xs, ws, n, 1)[0] == lanes[0]


# ------------------------------------------------------------------------------------------------ A6 / A7 / A9 / A10

def test_swiglu_trap_silu_on_up_is_observable():
    g = O.gen_normal(4, 1, 256)
    u = O.gen_normal(4, 2, 256)
    h_good = np.array([O.lib().or_silu_mul(float(a), float(b)) for a, b in zip(g, u)])
    h_bad = np.array([O.lib().or_silu_mul(float(b), float(a)) for a, b in zip(g, u)])
    assert np.abs(h_good - h_bad).sum() / np.abs(h_good).sum() > 0.5
    want = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    assert np.max(np.abs(h_good - want)) < 1e-6 * max(1.0, np.abs(want).max())
    # the q8_1 of h is the quantiser applied to h
    assert np.array_equal(O.swiglu_q8(g, u), O.quant_q8_1(h_good.astype(np.float32)))


def test_combine_against_double_and_traps():
    rng_parts = O.gen_normal(31337, 1, 10 * 256).reshape(10, 256)
    w = np.abs(O.gen_normal(31337, 2, 10)) + 0.05
    w = (w / w.sum()).astype(np.float32)
    shared = 3.0 * O.gen_normal(31337, 3, 256)
    want = O.combine_double(rng_parts, w, shared)
    got = O.combine_dev(rng_parts, w, shared)
    assert O.rel_l1_rows(got[None], want[None])[0] <= 1e-6   # metal/src/moe_combine_parity.cpp:19
    unweighted = O.combine_double(rng_parts, np.ones(10, np.float32), shared)
    shared_weighted = O.combine_double(rng_parts, w, shared * w[0])
    assert O.rel_l1_rows(unweighted[None], want[None])[0] > 0.05
    assert O.rel_l1_rows(shared_weighted[None], want[None])[0] > 0.05
    assert O.rel_l1_rows(O.combine_dev(rng_parts, w, None)[None], want[None])[0] > 0.05


def test_dispatch_against_brute_force_sort():
    T, K, E = 97, 10, 64
    logits = O.gen_normal(1, 1, T * E).reshape(T, E)
    ids, _ = O.route_dev(logits, K)
    counts, offsets, perm, slot = O.dispatch(ids, E)
    flat = ids.ravel()
    assert counts.sum() == T * K and (counts == np.bincount(flat, minlength=E)).all()
    assert offsets[0] == 0 and (np.diff(offsets) == counts).all()
    want = np.argsort(flat, kind="stable")
    assert np.array_equal(perm, want)
    assert np.array_equal(slot[perm], np.arange(T * K))


# ------------------------------------------------------------------------------------------------ the whole block

def test_golden_layer_reproduces_bitwise():
    f = np.load(os.path.join(GOLD, "layer_small.npz"))
    H, F, Fs, E, K, wt, st, seed = [int(v) for v in f["geom"]]
    g = O.Geom(n_embd=H, n_ff=F, n_ff_shared=Fs, n_expert=E, top_k=K, w_type=wt, sh_type=st)
    w = O.make_weights(g, seed)
    for n in ("gate_exps", "up_exps", "down_exps", "router", "gate_sh", "up_sh", "down_sh", "gate_inp_sh"):
        assert sha(getattr(w, n)) == str(f["sha_" + n]), n
    y, tr = O.moe_decode_dev(g, w, f["x"], trace=True)
    assert np.array_equal(y.view(np.uint32), f["y"].view(np.uint32))
    for k in ("logits", "ids", "weights", "counts", "offsets", "perm", "slot", "sgate", "xq"):
        assert np.array_equal(tr[k], f[k]), k
    yp = O.moe_prefill(g, w, f["x"])
    assert np.array_equal(yp.view(np.uint32), np.load(os.path.join(GOLD, "layer_prefill.npz"))["y"].view(np.uint32))


def test_block_device_order_vs_reference_order_config1():
    g = O.Geom()
    w = O.make_weights(g, 1)
    x = O.gen_normal(11, 100, 2 * g.n_embd).reshape(2, g.n_embd)
    y, tr = O.moe_decode_dev(g, w, x, trace=True)
    yr = O.moe_decode_ref(g, w, x)
    assert O.rel_l1_rows(y, yr).max() <= 1e-3          # the north-star gate; measured ~1e-7
    assert O.rel_l1_rows(y, yr).max() <= 1e-5
    ids_r, w_r = O.route_ref(tr["logits"], g.top_k)     # stage-wise routing, metal/src/pack_parity.cpp:8626
    assert np.array_equal(ids_r, tr["ids"])
    # trap: dropping the shared expert moves the output (metal/src/pack_parity.cpp:8671-8677)
    y_noshared = O.moe_decode_dev(g, w, x, add_shared=False)
    assert O.rel_l1_rows(y_noshared, y).min() > 1e-3


def _exact_block(g, w, x, tr):
    """fp64 MoE over the dequantised weights and unrounded activations, with the given routing."""
    H, F, Fs, K = g.n_embd, g.n_ff, g.n_ff_shared, g.top_k
    deq = lambda b, r, c: O.dequant_q2_0(b).reshape(-1, r, c).astype(np.float64)  # noqa: E731
    gate, up, down = deq(w.gate_exps, F, H), deq(w.up_exps, F, H), deq(w.down_exps, H, F)
    gs, us, ds = deq(w.gate_sh, Fs, H)[0], deq(w.up_sh, Fs, H)[0], deq(w.down_sh, H, Fs)[0]
    silu = lambda v: v / (1 + np.exp(-v))  # noqa: E731
    y = np.zeros((x.shape[0], H))
    for t in range(x.shape[0]):
        xt = x[t].astype(np.float64)
        for s in range(K):
            e = tr["ids"][t, s]
            y[t] += tr["weights"][t, s] * (down[e] @ (silu(gate[e] @ xt) * (up[e] @ xt)))
        gi = O.f32_from_bf16(w.gate_inp_sh).astype(np.float64) @ O.f32_from_bf16(O.bf16_from_f32(x[t]))
        y[t] += (ds @ (silu(gs @ xt) * (us @ xt))) / (1 + np.exp(-gi))
    return y


def test_contract_deviation_from_exact_fp64():
    """Both contracts against an fp64 evaluation of the same routed experts.  The decode contract is the
    reference's q8_1 one (metal/shaders/iq.metal:597-627) and carries its ~3% activation-rounding error; the
    prefill contract (bf16 activations, exact block scales) is ~0.5%.  Parity is gated within a contract."""
    g = O.Geom(n_embd=512, n_ff=256, n_ff_shared=256, n_expert=32, top_k=4)
    w = O.make_weights(g, 77)
    x = O.gen_normal(77, 100, 4 * g.n_embd).reshape(4, g.n_embd)
    yd, td = O.moe_decode_dev(g, w, x, trace=True)
    yp, tp = O.moe_prefill(g, w, x, trace=True)
    assert np.array_equal(td["ids"], tp["ids"])          # routing is the same A5 router in both
    ye = _exact_block(g, w, x, td)
    assert O.rel_l1_rows(yp, ye).max() < 1e-2
    assert O.rel_l1_rows(yd, ye).max() < 6e-2


def _prefill_contract_fp64(g, w, x, tr, round_x=True, round_h=True):
    """The prefill contract evaluated independently in fp64 from the pinned pieces: weights dequantised by
    or_dequant_q2_0 (pinned against the reference's vectors), activations and h rounded by numpy's bf16 rule
    (pinned against the reference's codec), SwiGLU and the sigmoid in fp64, the combine in fp64."""
    H, F, Fs, K = g.n_embd, g.n_ff, g.n_ff_shared, g.top_k
    deq = lambda b, r, c: O.dequant_q2_0(b).reshape(-1, r, c).astype(np.float64)  # noqa: E731
    gate, up, down = deq(w.gate_exps, F, H), deq(w.up_exps, F, H), deq(w.down_exps, H, F)
    gs, us, ds = deq(w.gate_sh, Fs, H)[0], deq(w.up_sh, Fs, H)[0], deq(w.down_sh, H, Fs)[0]
    b16 = lambda v: O.f32_from_bf16(O.bf16_from_f32(np.asarray(v, np.float32))).astype(np.float64)  # noqa: E731
    silu = lambda v: v / (1 + np.exp(-v))  # noqa: E731
    y = np.zeros((x.shape[0], H))
    for t in range(x.shape[0]):
        xt = b16(x[t]) if round_x else x[t].astype(np.float64)
        for s in range(K):
            e = tr["ids"][t, s]
            h = silu((gate[e] @ xt).astype(np.float32)) * (up[e] @ xt).astype(np.float32)
            h = b16(h) if round_h else h
            y[t] += float(tr["weights"][t, s]) * (down[e] @ h)
        h = silu((gs @ xt).astype(np.float32)) * (us @ xt).astype(np.float32)
        h = b16(h) if round_h else h
        y[t] += (ds @ h) / (1 + np.exp(-float(tr["sgate"][t])))
    return y


def test_prefill_oracle_beyond_the_fp16_operand_limit():
    """The prefill contract itself has no fp16 limit: a token whose activations reach 1e5 (beyond the device's fp16
    MFMA operands, which the trace's overflow mask reports) stays finite in the oracle, and the other tokens are as
    without it."""
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4)
    w = O.make_weights(g, 31)
    x = O.gen_normal(31, 100, 6 * 256).reshape(6, 256)
    y = O.moe_prefill(g, w, x)
    xb = x.copy()
    xb[2] *= 1e5
    yb = O.moe_prefill(g, w, xb)
    assert np.isfinite(yb).all() and np.abs(yb[2]).max() > 65520.0
    keep = np.arange(6) != 2
    assert np.array_equal(yb[keep].view(np.uint32), y[keep].view(np.uint32))


def test_prefill_oracle_against_independent_fp64_contract():
    """or_moe_prefill (the GPU MFMA path's checker) against the contract evaluated in fp64 from pinned pieces:
    within 1e-5 per row.  Dropping either bf16 rounding (x or h) moves the result by ~1e-3, so both traps are
    caught; routing is the pinned A5 router."""
    g = O.Geom(n_embd=512, n_ff=256, n_ff_shared=256, n_expert=32, top_k=4)
    w = O.make_weights(g, 78)
    x = O.gen_normal(78, 100, 6 * g.n_embd).reshape(6, g.n_embd)
    yp, tp = O.moe_prefill(g, w, x, trace=True)
    want = _prefill_contract_fp64(g, w, x, tp)
    assert O.rel_l1_rows(yp, want).max() < 1e-5
    for kw in (dict(round_x=False), dict(round_h=False)):
        trap = _prefill_contract_fp64(g, w, x, tp, **kw)
        assert O.rel_l1_rows(yp, trap).max() > 1e-4, kw


@pytest.mark.parametrize("n", [2048, 2560, 128, 300])
def test_residual_rmsnorm_pinned(n):
    """The stacked configuration's junction RMSNorm(x + r): against the float64 formula, the closed form of a
    constant row, and (eps = 0) exact invariance under a power-of-two scale of the input."""
    x = O.gen_normal(8, n, 4 * n).reshape(4, n)
    r = O.gen_normal(8, n + 1, 4 * n).reshape(4, n)
    y = O.residual_rmsnorm_dev(x, r)
    s = x.astype(np.float64) + r
    ref = s / np.sqrt((s * s).mean(-1, keepdims=True) + 1e-6)
    assert np.abs(y - ref).max() <= 1e-6 * np.abs(ref).max()
    y0 = O.residual_rmsnorm_dev(x)  # r = NULL: RMSNorm(x)
    ref0 = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6)
    assert np.abs(y0 - ref0).max() <= 1e-6 * np.abs(ref0).max()
    c = np.full((1, n), 0.75, np.float32)
    assert np.allclose(O.residual_rmsnorm_dev(c), 0.75 / np.sqrt(0.5625 + 1e-6), rtol=2e-7, atol=0)
    a = O.residual_rmsnorm_dev(x, r, eps=0.0)
    b = O.residual_rmsnorm_dev(4 * x, 4 * r, eps=0.0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_cpu_pool_baseline_equals_device_order_oracle():
    """The timed CPU baseline (oracle/smoe_cpu_pool.c: the decode contract in (expert, row-range) job batches,
    weight rows decoded once per expert for all of its tokens) is bitwise the device-order oracle it restates, for
    both weight types, with and without the shared expert, on one thread and several."""
    for wt, H, F in ((O.Q2_0, 256, 128), (O.Q2_0, 512, 384), (O.IQ2_S, 512, 512)):
        for sh in (wt, -1):
            g = O.Geom(n_embd=H, n_ff=F, n_ff_shared=F, n_expert=16, top_k=4, w_type=wt, sh_type=sh)
            w = O.make_weights(g, 11 + H)
            for T in (1, 3, 9):
                x = O.gen_normal(3, 100 + T, T * H).reshape(T, H)
                want = O.moe_decode_dev(g, w, x)
                for th in (1, 4):
                    got = O.moe_decode_pool(g, w, x, n_threads=th)
                    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (wt, H, sh, T, th)
    # a shared expert wider than the routed ones, and add_shared off
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=256, n_expert=8, top_k=2)
    w = O.make_weights(g, 5)
    x = O.gen_normal(4, 1, 5 * 256).reshape(5, 256)
    for add in (True, False):
        assert np.array_equal(O.moe_decode_pool(g, w, x, add_shared=add, n_threads=3).view(np.uint32),
                              O.moe_decode_dev(g, w, x, add_shared=add).view(np.uint32))
    # the f32 router (router_dtype 1)
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4, router_dtype=1)
    w = O.make_weights(g, 6)
    assert w.router.dtype == np.float32
    x = O.gen_normal(4, 2, 3 * 256).reshape(3, 256)
    want = O.moe_decode_dev(g, w, x)
    assert np.array_equal(O.moe_decode_pool(g, w, x, n_threads=2).view(np.uint32), want.view(np.uint32))
    # and the router type is observable: the bf16 router of the same generator routes differently somewhere
    gb = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4)
    assert not np.array_equal(O.moe_decode_dev(gb, O.make_weights(gb, 6), x).view(np.uint32), want.view(np.uint32))
