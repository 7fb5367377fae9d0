"""The reference's stage-wise check of one MoE pass (walk_ffn, metal/src/pack_parity.cpp:8584-8600 and
8764-8770), applied to a device trace that carries the expert stages.

Every stage is recomputed on the host, in the reference's order, from the device's own input to that stage, and must
agree within the reference's bounds (rel_l1):
- router logits against a double dot (1e-5), and the shared gate dot (1e-4, the reference's bound for it);
- each routed pair's gate and up dots from the device's q8_1 of x (1e-5), its down row from the device's q8_1 of h
  (1e-5);
- the shared expert's gate and up from the device's q8_1 of x (1e-5), its down from the device's q8_1 of its h, times
  sigmoid of the device's gate dot (1e-5);
- the combine: a double sum of the device's parts and shared rows with the device's weights (1e-5).
When those hold, an output row can differ from the reference-order chain only where an int8 of h (or a block scale)
quantises to the neighbouring q8_1 step from the reference order's f32 values: `flips` names every such value.
"""
from dataclasses import dataclass, field
from typing import Dict, List

import numpy as np

import oracle as O

BOUND = 1e-5
# the shared gate is one dot per token: the reference bounds it (its `scale`) at 1e-4 (pack_parity.cpp:8764)
BOUNDS = {"shared gate dot": 1e-4}


def rel_l1(got, want) -> float:
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    den = np.abs(want).sum()
    num = np.abs(got - want).sum()
    return float(num / den) if den > 0 else (0.0 if num == 0 else 1.0)


def q8_blocks(b: np.ndarray):
    """(d, q) of a run of 36-byte q8_1 blocks: the fp16 scale as f32 and the 32 int8 values of each block."""
    b = np.ascontiguousarray(b, np.uint8).reshape(-1, 36)
    d = O.f32_from_f16(b[:, 0:2].copy().view(np.uint16).ravel())
    q = b[:, 4:36].copy().view(np.int8)
    return d, q


@dataclass
class Flip:
    row: int        # pair row (dispatch position), or -1 - t for the shared expert's token t
    token: int
    expert: int     # -1: the shared expert
    index: int      # value of h
    dev: int        # the device's int8 (times its block scale below)
    ref: int        # the reference order's int8
    d_dev: float
    d_ref: float


@dataclass
class Report:
    worst: Dict[str, float] = field(default_factory=dict)
    flips: List[Flip] = field(default_factory=list)

    def note(self, name: str, v: float):
        self.worst[name] = max(self.worst.get(name, 0.0), v)

    def ok(self) -> bool:
        return all(v <= BOUNDS.get(k, BOUND) for k, v in self.worst.items())

    def summary(self) -> str:
        s = ", ".join(f"{k} {v:.2e}" for k, v in sorted(self.worst.items()))
        return f"{s}; {len(self.flips)} h value(s) on the other q8_1 step"

    def flipped_tokens(self):
        return sorted({f.token for f in self.flips})


def _gemv_ref(wtype: int):
    if wtype == O.Q2_0:
        return O.q2_0_gemv_ref
    if wtype == O.IQ2_S:
        return O.iq2_s_gemv_ref
    return lambda w, xq, n_in, n_out: O.native_gemv(wtype, w, xq, n_in, n_out)[0]  # the reference's 32-lane order


def _h_flips(rep: Report, row: int, token: int, expert: int, g_ref, u_ref, hq_dev):
    """The values of h whose q8_1 differs between the device's block and the quantisation of the reference-order
    gate and up."""
    d_ref, q_ref = q8_blocks(O.swiglu_q8(g_ref, u_ref))
    d_dev, q_dev = q8_blocks(hq_dev)
    for b, i in zip(*np.nonzero((q_ref != q_dev) | (d_ref != d_dev)[:, None])):
        rep.flips.append(Flip(row, token, expert, int(b * 32 + i), int(q_dev[b, i]), int(q_ref[b, i]),
                              float(d_dev[b]), float(d_ref[b])))


def stagewise(g: "O.Geom", w: "O.Weights", x: np.ndarray, tr: Dict[str, np.ndarray], y: np.ndarray,
              add_shared: bool) -> Report:
    """The stage-wise check of a traced decode-path pass (`tr`: host copies of the trace with stages)."""
    x = np.asarray(x, np.float32)
    T, H = x.shape
    F, Fs, E, K = g.n_ff, g.n_ff_shared, g.n_expert, g.top_k
    rep = Report()
    xq = np.asarray(tr["xq"]).reshape(T, H // 32 * 36)
    # the router and the shared gate from the device's bf16 of x (the reference: bf16_dot of the rounded mix)
    xb = O.bf16_from_f32(x)
    for t in range(T):
        if g.router_dtype == 1:
            lg = O.f32_gemv_double(x[t], w.router, H, E)
        else:
            lg = O.bf16_gemv_double(xb[t], w.router, H, E)
        if w.logit_bias is not None:
            lg = lg + w.logit_bias.astype(np.float64)
        rep.note("router", rel_l1(tr["logits"][t], lg))
        if g.sh_type >= 0:
            sgr = O.bf16_gemv_double(xb[t], w.gate_inp_sh, H, 1)
            rep.note("shared gate dot", rel_l1(tr["sgate"][t:t + 1], sgr))
    # routed pairs, by dispatch position
    ids = np.asarray(tr["ids"]).reshape(T, K)
    perm = np.asarray(tr["perm"]).ravel()
    slot = np.asarray(tr["slot"]).ravel()
    wts = np.asarray(tr["weights"]).reshape(T, K)
    hq = np.asarray(tr["hq"]).reshape(T * K, F // 32 * 36)
    egate = np.asarray(tr["egate"]).reshape(T * K, F)
    eup = np.asarray(tr["eup"]).reshape(T * K, F)
    parts = np.asarray(tr["parts"]).reshape(T * K, H)
    rb_in, rb_ff = O.row_bytes(g.w_type, H), O.row_bytes(g.w_type, F)
    ref = _gemv_ref(g.w_type)
    for p in range(T * K):
        pair = int(perm[p])
        t, e = pair // K, int(ids.ravel()[pair])
        G = w.gate_exps[e * F * rb_in:(e + 1) * F * rb_in]
        U = w.up_exps[e * F * rb_in:(e + 1) * F * rb_in]
        D = w.down_exps[e * H * rb_ff:(e + 1) * H * rb_ff]
        g_ref, u_ref = ref(G, xq[t], H, F), ref(U, xq[t], H, F)
        rep.note("expert gate", rel_l1(egate[p], g_ref))
        rep.note("expert up", rel_l1(eup[p], u_ref))
        rep.note("expert down", rel_l1(parts[p], ref(D, hq[p], F, H)))
        _h_flips(rep, p, t, e, g_ref, u_ref, hq[p])
    # the shared expert
    shared = None
    if g.sh_type >= 0:
        tg, tu, td = g.shared_types()
        shared = np.asarray(tr["shared"]).reshape(T, H)
        sgu = np.asarray(tr["sgu"]).reshape(2, T, -1)[:, :, :Fs]
        shq = np.asarray(tr["shq"]).reshape(T, -1)[:, :Fs // 32 * 36]
        sig = 1.0 / (1.0 + np.exp(-np.asarray(tr["sgate"], np.float64).ravel()))
        for t in range(T):
            g_ref = _gemv_ref(tg)(w.gate_sh, xq[t], H, Fs)
            u_ref = _gemv_ref(tu)(w.up_sh, xq[t], H, Fs)
            rep.note("shared gate", rel_l1(sgu[0, t], g_ref))
            rep.note("shared up", rel_l1(sgu[1, t], u_ref))
            d_ref = np.asarray(_gemv_ref(td)(w.down_sh, shq[t], Fs, H), np.float64) * sig[t]
            rep.note("shared down", rel_l1(shared[t], d_ref))
            _h_flips(rep, -1 - t, t, -1, g_ref, u_ref, shq[t])
    # the combine in double from the device's rows
    for t in range(T):
        acc = np.zeros(H, np.float64)
        for s in range(K):
            acc += float(wts[t, s]) * parts[slot[t * K + s]].astype(np.float64)
        if shared is not None and add_shared:
            acc += shared[t]
        rep.note("combine", rel_l1(y[t], acc))
    return rep


def reference_order_gate(g, w, x, y, add_shared, run_stages, say=print, n_threads=8):
    """north_star's gate against the reference's host chain: every output row within 1e-3 (rel_l1) of the
    reference-order chain, or, for a row beyond it, the reference's own stage-wise check on the device's inputs
    (run_stages() -> host trace with stages) passes and names the h values behind the row.  Returns the per-row
    relative errors."""
    yref = O.moe_decode_ref(g, w, x, add_shared=add_shared, n_threads=n_threads)
    rel = O.rel_l1_rows(y, yref)
    over = np.nonzero(rel > 1e-3)[0]
    if over.size:
        tr, y_st = run_stages()
        assert np.array_equal(np.asarray(y_st).view(np.uint32), np.asarray(y).view(np.uint32)), \
            "the traced pass gave other bits"
        rep = stagewise(g, w, x, tr, y, add_shared)
        say(f"  rows beyond 1e-3 of the reference order: {over.tolist()} (max {rel.max():.3e}); "
            f"stage-wise: {rep.summary()}")
        for f in rep.flips:
            if f.token in set(over.tolist()):
                say(f"    token {f.token} {'shared' if f.expert < 0 else f'expert {f.expert}'} h[{f.index}]: "
                    f"device {f.dev} x {f.d_dev:.6g}, reference order {f.ref} x {f.d_ref:.6g}")
        assert rep.ok(), f"stage-wise check failed: {rep.summary()}"
        missing = sorted(set(over.tolist()) - set(rep.flipped_tokens()))
        assert not missing, f"rows {missing} beyond 1e-3 with no h value on the other q8_1 step"
    return rel
