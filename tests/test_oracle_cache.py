"""The expert tier without a GPU: the oracle's hit/miss split and grouping (oracle/smoe_cache.c) pinned against an
independent statement of the same lists, or_expert_dev pinned against the block oracle's routed pair rows, and the
C ABI's refusals of smoe_expert_group / smoe_expert_grouped / smoe_verify_* before any launch.

The reference states the split's contract (include/strata/kernels/s2_expert_grouped.hpp:92-112: a hit list from the
routed ids and a residency row, hit rows landing on their routed indices, groups with one blob each) but its kernels
are not in the reference tree; the order of groups and entries is this library's (ascending expert id, then
ascending routing index), and the independent statement below is a sort of the hit indices by that key."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
import stratametal_amd as S

FAKE = 0x10000000


def split_by_sort(ids, kpt, E, resident):
    """The same lists from Python's sort: hits keyed (expert, index), misses in index order."""
    ids = [int(v) for v in np.asarray(ids).ravel()]
    hit = [i for i, e in enumerate(ids) if 0 <= e < E and resident[e]]
    miss = [i for i, e in enumerate(ids) if not (0 <= e < E and resident[e])]
    hit.sort(key=lambda i: (ids[i], i))
    experts = sorted({ids[i] for i in hit})
    starts, at = [], 0
    for e in experts:
        starts.append(at)
        at += sum(1 for i in hit if ids[i] == e)
    starts.append(at)
    return experts, starts, hit, [i // kpt for i in hit], miss


CASES = [(0, 1, 4), (1, 1, 4), (7, 3, 8), (128, 10, 512), (1000, 10, 512), (4096, 8, 1024), (300, 4, 16)]


@pytest.mark.parametrize("n,kpt,E", CASES)
@pytest.mark.parametrize("frac", [0.0, 0.3, 1.0])
def test_expert_group_matches_sort(n, kpt, E, frac):
    rng = np.random.default_rng(n * 7 + kpt + int(frac * 10))
    ids = rng.integers(0, E, n).astype(np.int32)
    if n > 4:  # ids outside the table are misses
        ids[rng.integers(0, n, 3)] = np.array([-1, E, 1 << 20], np.int32)
    resident = (rng.random(E) < frac).astype(np.uint8)
    r = O.expert_group(ids, kpt, E, resident)
    experts, starts, dst, tok, miss = split_by_sort(ids, kpt, E, resident)
    ng, nh, nm = (int(v) for v in r["counts"][:3])
    assert (ng, nh, nm) == (len(experts), len(dst), len(miss))
    assert list(r["grp_expert"][:ng]) == experts and list(r["grp_start"][:ng + 1]) == starts
    assert list(r["ent_dst"][:nh]) == dst and list(r["ent_tok"][:nh]) == tok
    assert list(r["miss_dst"][:nm]) == miss


def test_expert_group_invariants():
    """Every entry exactly once (hit or miss), each group's entries of its expert and resident, misses not."""
    rng = np.random.default_rng(11)
    E, kpt = 64, 6
    for trial in range(20):
        n = int(rng.integers(1, 600))
        ids = rng.integers(-2, E + 2, n).astype(np.int32)
        res = (rng.random(E) < rng.random()).astype(np.uint8)
        r = O.expert_group(ids, kpt, E, res)
        ng, nh, nm = (int(v) for v in r["counts"][:3])
        both = np.concatenate([r["ent_dst"][:nh], r["miss_dst"][:nm]])
        assert np.array_equal(np.sort(both), np.arange(n))
        for g in range(ng):
            a, b = r["grp_start"][g], r["grp_start"][g + 1]
            e = r["grp_expert"][g]
            assert b > a and res[e] and np.all(ids[r["ent_dst"][a:b]] == e)
            assert np.all(np.diff(r["ent_dst"][a:b]) > 0)
        assert np.all(np.diff(r["grp_expert"][:ng]) > 0)
        for i in r["miss_dst"][:nm]:
            assert not (0 <= ids[i] < E and res[ids[i]])
        assert np.array_equal(r["ent_tok"][:nh], r["ent_dst"][:nh] // kpt)


@pytest.mark.parametrize("wtype", [O.Q2_0, O.IQ2_S])
def test_expert_dev_is_the_block_oracles_pair_row(wtype):
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=8, top_k=3) if wtype == O.Q2_0 else \
        O.Geom(n_embd=512, n_ff=512, n_ff_shared=512, n_expert=8, top_k=3, w_type=O.IQ2_S, sh_type=O.IQ2_S)
    w = O.make_weights(g, 5)
    T = 3
    x = O.gen_normal(5, 9, T * g.n_embd).reshape(T, g.n_embd)
    _, tr = O.moe_decode_dev(g, w, x, trace=True)
    xq = O.quant_q8_1(x).reshape(T, -1)
    for i in range(T * g.top_k):
        e, t = int(tr["ids"].ravel()[i]), i // g.top_k
        row = O.expert_dev(wtype, O.expert_blob(g, w, e), g.n_embd, g.n_ff, xq[t])
        assert np.array_equal(row.view(np.uint32), tr["parts"][tr["slot"][i]].view(np.uint32)), i


def test_expert_dev_sees_the_blob_order():
    """Swapping the gate and up halves of a blob changes the row (the chain reads gate first, SwiGLU is not
    symmetric)."""
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=4, top_k=2)
    w = O.make_weights(g, 6)
    b = O.expert_blob(g, w, 1)
    gu = len(w.gate_exps) // g.n_expert
    sw = np.concatenate([b[gu:2 * gu], b[:gu], b[2 * gu:]])
    xq = O.quant_q8_1(O.gen_normal(6, 1, g.n_embd))
    assert not np.array_equal(O.expert_dev(O.Q2_0, b, 256, 128, xq), O.expert_dev(O.Q2_0, sw, 256, 128, xq))


# ---- refusals before any launch (no GPU needed; the fake pointers are never dereferenced)

def test_expert_group_refusals():
    L = S.lib()
    args = lambda n=4, kpt=2, E=8, table=FAKE: (FAKE, n, kpt, E, table, FAKE, FAKE, None, FAKE, FAKE, FAKE, FAKE, None)
    assert L.smoe_expert_group(*args(n=4097)) == -1
    assert L.smoe_expert_group(*args(n=-1)) == -1
    assert L.smoe_expert_group(*args(kpt=0)) == -1
    assert L.smoe_expert_group(*args(E=0)) == -1
    assert L.smoe_expert_group(*args(E=1025)) == -1
    assert L.smoe_expert_group(*args(table=None)) == -6
    assert L.smoe_expert_group(*args(table=FAKE + 4)) == -5


def test_expert_grouped_and_verify_refusals():
    L = S.lib()
    g = S.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=8, top_k=2)
    gc = g.c()
    assert L.smoe_expert_blob_bytes(C.byref(gc)) == 2 * 128 * (256 // 64 * 18) + 256 * (128 // 64 * 18)
    assert L.smoe_expert_blob_bytes(C.byref(S.Geom(n_embd=100).c())) == 0
    ws = L.smoe_expert_grouped_workspace_bytes(C.byref(gc), 4, 8, 16)
    assert ws > 0
    call = lambda cg=8, ce=16, T=4, wsb=ws, out=FAKE, x=FAKE, ws_p=FAKE: L.smoe_expert_grouped(
        C.byref(gc), FAKE, FAKE, FAKE, FAKE, FAKE, cg, ce, x, T, out, 8, ws_p, wsb, None)
    assert call(cg=-1) == -1
    assert call(cg=65536) == -1  # one grid row per group: at most 65535
    assert call(ce=(1 << 24) + 1) == -1
    assert call(wsb=ws - 1) == -2
    assert call(out=None) == -6
    assert call(ws_p=FAKE + 64) == -5
    assert call(T=0) == 0 and call(cg=0) == 0  # nothing to do: no launch
    assert L.smoe_expert_grouped(C.byref(S.Geom(w_type=7).c()), FAKE, FAKE, FAKE, FAKE, FAKE, 8, 16, FAKE, 4, FAKE, 8,
                                 FAKE, ws, None) == -3
    # the verify window
    assert L.smoe_verify_workspace_bytes(C.byref(gc), 16) > 0
    assert L.smoe_verify_workspace_bytes(C.byref(gc), 2049) == 0  # T * k > 4096
    vws = L.smoe_verify_workspace_bytes(C.byref(gc), 4)
    w = S._Weights(*([FAKE] * 8 + [None]))
    begin = lambda T=4, table=FAKE, wsb=vws, rows=FAKE, ww=w: L.smoe_verify_begin(
        C.byref(gc), C.byref(ww), table, FAKE, T, rows, FAKE, FAKE, FAKE, FAKE, FAKE, wsb, None)
    assert begin(T=-1) == -1
    assert begin(T=3000) == -1
    assert begin(T=0) == 0
    assert begin(table=None) == -6
    assert begin(wsb=vws - 1) == -2
    assert begin(table=FAKE + 4) == -5
    assert begin(rows=FAKE + 16) == -1  # rows overlaps x
    assert begin(ww=S._Weights(*([FAKE] * 3 + [None] + [FAKE] * 4 + [None]))) == -6
    end = lambda T=4, wsb=vws, y=FAKE + (1 << 24): L.smoe_verify_end(C.byref(gc), T, FAKE, FAKE, 1, y, FAKE, wsb,
                                                                     None)
    assert end(T=-1) == -1 and end(T=0) == 0
    assert end(wsb=vws - 1) == -2
    assert end(y=FAKE) == -1  # y overlaps rows


def test_python_binding_refuses_short_lists():
    """The grouped-experts and verify-window bindings refuse, before any launch, lists shorter than the caps and
    activations of the wrong width (CPU tensors: the size checks come before the device check)."""
    import torch
    g = S.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=8, top_k=2)
    groups = dict(grp_ptr=torch.zeros(4, dtype=torch.int64), grp_start=torch.zeros(5, dtype=torch.int32),
                  ent_dst=torch.zeros(8, dtype=torch.int32), ent_tok=torch.zeros(8, dtype=torch.int32),
                  counts=torch.zeros(4, dtype=torch.int32))
    x = torch.zeros(4 * (256 // 32) * 36, dtype=torch.uint8)
    out = torch.zeros((8, 256), dtype=torch.float32)
    with pytest.raises(S.SmoeError, match="grp_ptr has 4 elements, needs 5"):
        S.expert_grouped(g, groups, x, 4, out, cap_groups=5)
    with pytest.raises(S.SmoeError, match="ent_tok has 8 elements, needs 9"):
        S.expert_grouped(g, dict(groups, ent_dst=torch.zeros(9, dtype=torch.int32)), x, 4, out)
    with pytest.raises(S.SmoeError, match="out has shape"):
        S.expert_grouped(g, groups, x, 4, torch.zeros((8, 128), dtype=torch.float32))
