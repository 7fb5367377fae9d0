"""Checks of the prefill path's router, stage by stage (the reference's method: metal/src/router_parity.cpp:21 bounds
the logits at 1e-5 against a double sum, metal/src/pack_parity.cpp:8626 routes the device's own logits on the host).

The prefill path's router runs on the matrix cores from 128 tokens: its logits are exact bf16 products summed in the
matrix core's f32 order, so they are compared with the exact dot (a double sum, bias added) within 1e-5 rel_l1 per
token, and the routing and dispatch must be exactly the device order's of those logits.  The block's output is then
compared with the prefill contract routed from the same logits (oracle.moe_prefill with logits given).
"""
import numpy as np

import oracle as O

LOGIT_BOUND = 1e-5
# The shared gate is one dot per token, which can sit near zero: its error is bounded against the magnitude of its
# products, |sg - exact| <= SGATE_BOUND * sum |x_h w_h| (f32 sums of 2048 products stay near 3e-6 of it).
SGATE_BOUND = 1e-5


def _rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.abs(b).sum()
    return float(np.abs(a - b).sum() / den) if den > 0 else float(np.abs(a - b).sum())


def exact_logits(g, w, x):
    """[T][E] exact router dots of bf16 x (f32 x for an f32 router) in double, plus the bias; [T] shared gate dots and
    [T] the sums of their products' magnitudes."""
    x = np.asarray(x, np.float32)
    T, H = x.shape
    xb = O.bf16_from_f32(x)
    lg = np.empty((T, g.n_expert), np.float64)
    sg = np.zeros(T, np.float64)
    sgl1 = np.zeros(T, np.float64)
    if g.sh_type >= 0:
        wg = O.f32_from_bf16(w.gate_inp_sh).astype(np.float64)
    for t in range(T):
        if g.router_dtype == 1:
            lg[t] = O.f32_gemv_double(x[t], w.router, H, g.n_expert)
        else:
            lg[t] = O.bf16_gemv_double(xb[t], w.router, H, g.n_expert)
        if g.sh_type >= 0:
            p = O.f32_from_bf16(xb[t]).astype(np.float64) * wg
            sg[t] = p.sum()
            sgl1[t] = np.abs(p).sum()
    if w.logit_bias is not None:
        lg += w.logit_bias.astype(np.float64)
    return lg, sg, sgl1


def router_stagewise(g, w, x, tr, rows=None):
    """The device's router and routing from a host copy of its trace (logits, ids, weights, counts, offsets, perm,
    slot, sgate): logits within LOGIT_BOUND of the exact dot per token (the tokens `rows`, default all), the shared
    gate within SGATE_BOUND, ids, weights and the dispatch of every token exactly the device order's of the device's
    logits.  Returns the worst logit rel_l1."""
    lg = np.asarray(tr["logits"], np.float32)
    rows = np.arange(lg.shape[0]) if rows is None else np.asarray(rows)
    want, sg, sgl1 = exact_logits(g, w, np.asarray(x)[rows])
    worst = max(_rel(lg[t], want[i]) for i, t in enumerate(rows))
    assert worst <= LOGIT_BOUND, f"router logits {worst:.3e} from the exact dot"
    if g.sh_type >= 0:
        dev_sg = np.asarray(tr["sgate"], np.float64)[rows]
        ws = (np.abs(dev_sg - sg) / np.maximum(sgl1, 1e-30)).max()
        assert ws <= SGATE_BOUND, f"shared gate {ws:.3e} of its products' magnitude from the exact dot"
    ids, wts = O.route_dev(lg, g.top_k)
    assert np.array_equal(np.asarray(tr["ids"]).reshape(ids.shape), ids), "ids differ from the routing of the logits"
    assert np.array_equal(np.asarray(tr["weights"], np.float32).reshape(wts.shape).view(np.uint32),
                          wts.view(np.uint32)), "routing weights"
    counts, offsets, perm, slot = O.dispatch(ids, g.n_expert)
    for k, v in (("counts", counts), ("offsets", offsets), ("perm", perm), ("slot", slot)):
        assert np.array_equal(np.asarray(tr[k]).ravel(), v.ravel()), k
    return worst


def prefill_want(g, w, x, tr, rows=None, **kw):
    """The prefill contract routed from the device's own logits and shared gate dots (host copies in `tr`), for the
    tokens `rows` (default all; a token's output depends on its own row only)."""
    rows = slice(None) if rows is None else np.asarray(rows)
    return O.moe_prefill(g, w, np.asarray(x)[rows], logits=np.asarray(tr["logits"])[rows],
                         sgate=np.asarray(tr["sgate"])[rows] if g.sh_type >= 0 else None, **kw)
