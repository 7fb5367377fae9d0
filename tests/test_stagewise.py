"""The stage-wise checker (tests/stagewise.py) pinned on the CPU: fed the oracle's own device-order stages it passes,
and each planted mistake -- a down row off by 1e-4, two pairs' rows swapped, gate dots without the Q2_0 minus-one
term, a routing weight dropped from the combine, a shared down row without its sigmoid -- fails it.  The q8_1 flip
finder names exactly the values planted on the other step."""
import numpy as np
import pytest

import oracle as O
import stagewise as SW


def oracle_stages(g, w, x, add_shared=True):
    """A trace with the expert stages from the oracle's device order (what the GPU's traced pass returns)."""
    y, tr = O.moe_decode_dev(g, w, x, add_shared=add_shared, trace=True)
    T, H = x.shape
    F, Fs, K = g.n_ff, g.n_ff_shared, g.top_k
    xq = tr["xq"].reshape(T, H // 32 * 36)
    rb = O.row_bytes(g.w_type, H)
    egate = np.empty((T * K, F), np.float32)
    eup = np.empty((T * K, F), np.float32)
    for p in range(T * K):
        pair = int(tr["perm"][p])
        t, e = pair // K, int(tr["ids"].ravel()[pair])
        egate[p] = O.gemv_dev(g.w_type, w.gate_exps[e * F * rb:(e + 1) * F * rb], xq[t], H, F)
        eup[p] = O.gemv_dev(g.w_type, w.up_exps[e * F * rb:(e + 1) * F * rb], xq[t], H, F)
    tr["egate"], tr["eup"] = egate, eup
    if g.sh_type >= 0:
        sgu = np.empty((2, T, Fs), np.float32)
        for t in range(T):
            sgu[0, t] = O.gemv_dev(g.sh_type, w.gate_sh, xq[t], H, Fs)
            sgu[1, t] = O.gemv_dev(g.sh_type, w.up_sh, xq[t], H, Fs)
        tr["sgu"] = sgu
        tr["shq"] = O.swiglu_q8(sgu[0], sgu[1]).reshape(T, -1)
    return y, tr


@pytest.fixture(scope="module")
def case():
    g = O.Geom(n_embd=512, n_ff=256, n_ff_shared=256, n_expert=32, top_k=4)
    w = O.make_weights(g, 77)
    T = 3
    x = O.gen_normal(77, 100, T * g.n_embd).reshape(T, g.n_embd)
    y, tr = oracle_stages(g, w, x)
    return g, w, x, y, tr


def test_device_order_stages_pass(case):
    g, w, x, y, tr = case
    assert np.array_equal(O.swiglu_q8(tr["egate"], tr["eup"]), tr["hq"].ravel())
    rep = SW.stagewise(g, w, x, tr, y, True)
    assert rep.ok(), rep.summary()
    assert set(rep.worst) >= {"router", "expert gate", "expert up", "expert down", "shared gate", "shared up",
                              "shared down", "combine", "shared gate dot"}


def _fails(g, w, x, y, tr, name, **kw):
    rep = SW.stagewise(g, w, x, tr, y, True, **kw)
    assert not rep.ok(), f"{name} went unseen: {rep.summary()}"
    return rep


def test_planted_mistakes_fail(case):
    g, w, x, y, tr = case
    t2 = dict(tr)
    t2["parts"] = tr["parts"].copy()
    t2["parts"][1] *= np.float32(1.0 + 1e-4)
    assert _fails(g, w, x, y, t2, "down row off by 1e-4").worst["expert down"] > 1e-5
    t2 = dict(tr)
    t2["parts"] = tr["parts"].copy()
    t2["parts"][[0, 1]] = tr["parts"][[1, 0]]
    _fails(g, w, x, y, t2, "two pairs' rows swapped")
    t2 = dict(tr)
    rb = O.row_bytes(g.w_type, g.n_embd)
    xq = tr["xq"].reshape(x.shape[0], -1)
    eg = tr["egate"].copy()
    pair = int(tr["perm"][0])
    e = int(tr["ids"].ravel()[pair])
    eg[0] = O.q2_0_gemv_no_minus_one(w.gate_exps[e * g.n_ff * rb:(e + 1) * g.n_ff * rb], xq[pair // g.top_k],
                                     g.n_embd, g.n_ff)
    t2["egate"] = eg
    assert _fails(g, w, x, y, t2, "gate without the minus-one term").worst["expert gate"] > 1e-5
    t2 = dict(tr)
    t2["weights"] = tr["weights"].copy()
    t2["weights"][0, 2] = 0.0
    assert _fails(g, w, x, y, t2, "a weight dropped from the combine").worst["combine"] > 1e-5
    t2 = dict(tr)
    sg = tr["sgate"].astype(np.float64)
    t2["shared"] = (tr["shared"] / (1.0 / (1.0 + np.exp(-sg)))[:, None]).astype(np.float32)
    assert _fails(g, w, x, y, t2, "shared rows without the sigmoid").worst["shared down"] > 1e-5


def test_flip_finder_names_planted_values(case):
    g, w, x, y, tr = case
    rep = SW.Report()
    p = 2
    hq = tr["hq"].reshape(-1, g.n_ff // 32 * 36)[p].copy()
    blk = hq.reshape(-1, 36)
    q = blk[1, 4:36].view(np.int8)
    q[5] = q[5] + (1 if q[5] < 127 else -1)  # value 32 + 5 on the neighbouring step
    SW._h_flips(rep, p, 0, 9, tr["egate"][p], tr["eup"][p], hq)
    assert [(f.row, f.index) for f in rep.flips] == [(p, 37)]
    rep = SW.Report()
    SW._h_flips(rep, p, 0, 9, tr["egate"][p], tr["eup"][p], tr["hq"].reshape(-1, g.n_ff // 32 * 36)[p])
    assert rep.flips == []


def test_reference_order_gate_on_the_oracle():
    """The gate itself on a case whose device order and reference order differ beyond 1e-3 on a row (600 experts,
    n_ff 128): the over-1e-3 rows are explained by named h flips and the stage-wise check passes."""
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=600, top_k=10)
    w = O.make_weights(g, 27)
    T = 16
    x = O.gen_normal(27, 100, T * g.n_embd).reshape(T, g.n_embd)
    y, tr = oracle_stages(g, w, x)
    msgs = []
    rel = SW.reference_order_gate(g, w, x, y, True, lambda: (tr, y), msgs.append)
    assert rel.max() > 1e-3  # this case does exercise the stage-wise route
    assert any("beyond 1e-3" in m for m in msgs)
