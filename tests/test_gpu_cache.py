"""GPU parity of the expert tier through the C ABI (stratametal_amd/csrc/smoe_cache.hip, smoe_api.cpp): experts
addressed one blob pointer each, the hit/miss split, the grouped experts and the verify window.

- smoe_expert_pack: each blob is the oracle's [gate rows | up rows | down rows] of the expert.
- smoe_expert_group: the lists equal the oracle's (oracle/smoe_cache.c, pinned by tests/test_oracle_cache.py)
  element for element, over table sizes up to 1024 experts and 4096 entries, ids outside the table included; the
  group pointers are the table's.
- smoe_expert_grouped: each entry's row is or_expert_dev's bit for bit (the decode contract's routed pair row);
  rows no entry names are left as they were; caller-made lists with a token or a row out of range, or a group
  without a blob, write nothing for those entries.
- the verify window: with every expert in the table, smoe_verify_begin + smoe_verify_end give smoe_forward's y and
  the oracle's bitwise (ids and weights too); with part of the experts in the table, the misses computed by
  smoe_expert_grouped over a second table give the same y -- a hit and a miss make the same number.  Q2_0 and
  IQ2_S routed experts, a fused and a native shared expert, the full benchmark geometry."""
import sys

import numpy as np
import pytest

import oracle as O
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


def layer(torch, g, seed):
    w_host = O.make_weights(g, seed)
    routed_types = g.sh_type < 0 or all(t in (O.Q2_0, O.IQ2_S) for t in g.shared_types())
    w_dev = S.synth_layer(S.Geom(**vars(g)), seed) if routed_types else None
    if w_dev is None:  # native shared projections: the routed planes from the device generator, the rest uploaded
        base = S.Geom(**{k: v for k, v in vars(g).items() if k not in ("sh_gate_type", "sh_up_type", "sh_down_type")})
        base.sh_type = g.w_type
        w_dev = S.synth_layer(base, seed)
        for n in ("gate_sh", "up_sh", "down_sh"):
            w_dev[n] = dev(torch, getattr(w_host, n))
    return w_host, w_dev


def blobs(torch, g, w_dev, experts):
    """A slot arena holding the given experts' blobs, and the table (0 for the others)."""
    nb = S.expert_blob_bytes(S.Geom(**vars(g)))
    arena = torch.empty((max(len(experts), 1), nb), dtype=torch.uint8, device="cuda")
    ptrs = [0] * g.n_expert
    for s, e in enumerate(experts):
        S.pack_expert(S.Geom(**vars(g)), w_dev, e, arena[s])
        ptrs[e] = arena[s].data_ptr()
    return arena, torch.tensor(ptrs, dtype=torch.int64, device="cuda")


def test_pack_expert_layout(torch):
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=8, top_k=2)
    say("case: pack_expert")
    w_host, w_dev = layer(torch, g, 3)
    arena, _ = blobs(torch, g, w_dev, [0, 5, 7])
    for s, e in enumerate([0, 5, 7]):
        assert np.array_equal(host(torch, arena[s]), O.expert_blob(g, w_host, e))


GROUP_CASES = [(1, 1, 4, 1.0), (10, 5, 8, 0.5), (128, 10, 512, 0.3), (1000, 10, 512, 0.7), (4096, 8, 1024, 0.5),
               (4096, 1, 16, 1.0), (300, 4, 64, 0.0)]


@pytest.mark.parametrize("case", range(len(GROUP_CASES)))
def test_expert_group_matches_oracle(torch, case):
    n, kpt, E, frac = GROUP_CASES[case]
    say(f"case: expert_group n={n} kpt={kpt} E={E} frac={frac}")
    rng = np.random.default_rng(case)
    ids = rng.integers(0, E, n).astype(np.int32)
    if n > 8:
        ids[rng.integers(0, n, 3)] = np.array([-1, E, 1 << 20], np.int32)
    res = (rng.random(E) < frac).astype(np.uint8)
    table = torch.tensor([(0x1000 * (e + 1)) if res[e] else 0 for e in range(E)], dtype=torch.int64, device="cuda")
    got = S.expert_group(dev(torch, ids), kpt, E, table)
    want = O.expert_group(ids, kpt, E, res)
    c = host(torch, got["counts"])
    assert np.array_equal(c, want["counts"])
    ng, nh, nm = int(c[0]), int(c[1]), int(c[2])
    assert np.array_equal(host(torch, got["grp_expert"])[:ng], want["grp_expert"][:ng])
    assert np.array_equal(host(torch, got["grp_start"])[:ng + 1], want["grp_start"][:ng + 1])
    assert np.array_equal(host(torch, got["ent_dst"])[:nh], want["ent_dst"][:nh])
    assert np.array_equal(host(torch, got["ent_tok"])[:nh], want["ent_tok"][:nh])
    assert np.array_equal(host(torch, got["miss_dst"])[:nm], want["miss_dst"][:nm])
    assert np.array_equal(host(torch, got["grp_ptr"])[:ng], 0x1000 * (want["grp_expert"][:ng].astype(np.int64) + 1))


GEOMS = {
    "q2_0 small": dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4),
    "iq2_s": dict(n_embd=512, n_ff=512, n_ff_shared=512, n_expert=16, top_k=4, w_type=O.IQ2_S, sh_type=O.IQ2_S),
    "full": dict(n_expert=512, top_k=10),
}


@pytest.mark.parametrize("name,T", [("q2_0 small", 5), ("iq2_s", 6), ("full", 16)])
def test_expert_grouped_rows(torch, name, T):
    say(f"case: expert_grouped {name} T={T}")
    g = O.Geom(**GEOMS[name])
    w_host, w_dev = layer(torch, g, 21)
    x = O.gen_normal(21, 3, T * g.n_embd).reshape(T, g.n_embd)
    _, tr = O.moe_decode_dev(g, w_host, x, trace=True, n_threads=8)
    ids = tr["ids"].ravel()
    held = sorted(set(int(e) for e in ids))[::2] + [e for e in range(g.n_expert) if e not in set(ids)][:3]
    arena, table = blobs(torch, g, w_dev, held)
    groups = S.expert_group(dev(torch, ids), g.top_k, g.n_expert, table)
    xq = S.quantize_q8_1(dev(torch, x))
    P = T * g.top_k
    sentinel = np.uint32(0x7FC01234)  # a NaN no kernel writes
    out = torch.full((P + 2, g.n_embd), int(sentinel), dtype=torch.int32, device="cuda").view(torch.float32)
    S.expert_grouped(S.Geom(**vars(g)), groups, xq, T, out)
    got = host(torch, out).view(np.uint32)
    xqh = O.quant_q8_1(x).reshape(T, -1)
    hit = set(int(i) for i in host(torch, groups["ent_dst"])[:int(host(torch, groups["counts"])[1])])
    for i in range(P + 2):
        if i in hit:
            e, t = int(ids[i]), i // g.top_k
            want = O.expert_dev(g.w_type, O.expert_blob(g, w_host, e), g.n_embd, g.n_ff, xqh[t])
            assert np.array_equal(got[i], bits(want)), i
            assert np.array_equal(got[i], bits(tr["parts"][tr["slot"][i]])), i
        else:
            assert np.all(got[i] == sentinel), f"row {i} (no entry) was written"


def test_expert_grouped_checks_caller_lists(torch):
    """Caller-made lists: an entry with a token or a row out of range and a group without a blob write nothing;
    the well-formed entries are computed as usual."""
    say("case: expert_grouped malformed lists")
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=8, top_k=2)
    w_host, w_dev = layer(torch, g, 22)
    T = 3
    x = O.gen_normal(22, 3, T * g.n_embd).reshape(T, g.n_embd)
    arena, table = blobs(torch, g, w_dev, [1, 2, 3])
    tp = host(torch, table)
    # groups: expert 1 (entries 0..2), expert 2 (3..4), a group without a blob (5), expert 3 (6..7)
    grp_ptr = np.array([tp[1], tp[2], 0, tp[3]], np.int64)
    grp_start = np.array([0, 3, 5, 6, 8], np.int32)
    ent_tok = np.array([0, 1, 7, 2, -1, 0, 1, 2], np.int32)    # entry 2: token 7 >= T; entry 4: token -1
    ent_dst = np.array([0, 1, 2, 3, 4, 5, 9, 6], np.int32)     # entry 6: row 9 >= 8 rows
    counts = np.array([4, 8, 0, 0], np.int32)
    groups = dict(grp_ptr=dev(torch, grp_ptr), grp_start=dev(torch, grp_start), ent_tok=dev(torch, ent_tok),
                  ent_dst=dev(torch, ent_dst), counts=dev(torch, counts))
    out = torch.zeros((8, g.n_embd), dtype=torch.float32, device="cuda")
    S.expert_grouped(S.Geom(**vars(g)), groups, S.quantize_q8_1(dev(torch, x)), T, out, cap_groups=4, cap_entries=8)
    got = host(torch, out)
    xqh = O.quant_q8_1(x).reshape(T, -1)
    good = {0: (1, 0), 1: (1, 1), 3: (2, 2), 6: (3, 2)}  # row: (expert, token)
    for r in range(8):
        if r in good:
            e, t = good[r]
            want = O.expert_dev(O.Q2_0, O.expert_blob(g, w_host, e), g.n_embd, g.n_ff, xqh[t])
            assert np.array_equal(bits(got[r]), bits(want)), r
        else:
            assert not got[r].any(), f"row {r} was written"
    # counts past the cap and group bounds past cap_entries are clipped, not followed
    counts2 = dev(torch, np.array([99, 0, 0, 0], np.int32))
    groups["counts"] = counts2
    groups["grp_start"] = dev(torch, np.array([0, 3, 5, 6, 1 << 30], np.int32))
    out2 = torch.zeros((8, g.n_embd), dtype=torch.float32, device="cuda")
    S.expert_grouped(S.Geom(**vars(g)), groups, S.quantize_q8_1(dev(torch, x)), T, out2, cap_groups=4, cap_entries=8)
    assert np.array_equal(bits(host(torch, out2)), bits(got))


VERIFY = [
    # name, geometry, T list, seed
    ("q2_0 fused shared", dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4), (1, 3, 9), 31),
    ("iq2_s", GEOMS["iq2_s"], (1, 5), 32),
    ("q2_0 with a native shared expert", dict(n_expert=64, top_k=8, sh_type=O.Q3_K, sh_down_type=O.IQ4_NL), (2, 7),
     33),
    ("full geometry", GEOMS["full"], (1, 4, 16), 34),
    ("no shared expert, f32 router", dict(n_embd=256, n_ff=256, n_expert=32, top_k=6, sh_type=-1, router_dtype=1),
     (4,), 35),
]


@pytest.mark.parametrize("case", range(len(VERIFY)))
def test_verify_window(torch, case):
    name, gkw, Ts, seed = VERIFY[case]
    g = O.Geom(**gkw)
    sg = S.Geom(**vars(g))
    w_host, w_dev = layer(torch, g, seed)
    all_arena, all_table = blobs(torch, g, w_dev, list(range(g.n_expert)))
    half = list(range(0, g.n_expert, 2))
    rest = [e for e in range(g.n_expert) if e % 2]
    h_arena, h_table = blobs(torch, g, w_dev, half)
    m_arena, m_table = blobs(torch, g, w_dev, rest)
    vw = S.VerifyWindow(sg, w_dev, max_tokens=max(Ts))
    ml = S.MoELayer(sg, w_dev, max_tokens=max(Ts))
    for T in Ts:
        say(f"case: verify window {name} T={T}")
        x = O.gen_normal(seed, 200 + T, T * g.n_embd).reshape(T, g.n_embd)
        xd = dev(torch, x)
        want, wtr = O.moe_decode_dev(g, w_host, x, trace=True, n_threads=8)
        y_fwd = host(torch, ml.forward(xd))
        assert np.array_equal(bits(y_fwd), bits(want))
        # every expert held: no misses, the forward's y
        r = vw.begin(xd, all_table)
        assert np.array_equal(host(torch, r["ids"]), wtr["ids"]) and np.array_equal(bits(host(torch, r["weights"])),
                                                                                   bits(wtr["weights"]))
        assert list(host(torch, r["counts"])[:3]) == [len(set(wtr["ids"].ravel())), T * g.top_k, 0]
        y = host(torch, vw.end(r))
        assert np.array_equal(bits(y), bits(want)), f"max rel {O.rel_l1_rows(y, want).max()}"
        if g.sh_type >= 0:
            y0 = host(torch, vw.end(r, add_shared=False))
            w0, _ = O.moe_decode_dev(g, w_host, x, add_shared=False, trace=True, n_threads=8)
            assert np.array_equal(bits(y0), bits(w0))
        # half the experts held: the split is the oracle's, the misses from the second table give the same y
        r = vw.begin(xd, h_table)
        res = np.zeros(g.n_expert, np.uint8)
        res[half] = 1
        ws = O.expert_group(wtr["ids"].ravel(), g.top_k, g.n_expert, res)
        c = host(torch, r["counts"])
        assert np.array_equal(c, ws["counts"])
        assert np.array_equal(host(torch, r["miss_dst"])[:c[2]], ws["miss_dst"][:c[2]])
        rows_before = host(torch, r["rows"]).copy()
        for i in ws["miss_dst"][:c[2]]:
            assert not rows_before[i].any(), "a miss row was written by begin"
        misses = S.expert_group(r["ids"].view(-1), g.top_k, g.n_expert, m_table)
        assert int(host(torch, misses["counts"])[1]) == int(c[2])
        S.expert_grouped(sg, misses, S.quantize_q8_1(xd), T, r["rows"])
        y2 = host(torch, vw.end(r))
        assert np.array_equal(bits(y2), bits(want))
        # the rows are the oracle's pair rows by routing index
        rows = host(torch, r["rows"])
        P = T * g.top_k
        assert np.array_equal(bits(rows[:P]), bits(wtr["parts"][wtr["slot"]]))
        if g.sh_type >= 0:
            assert np.array_equal(bits(rows[P:P + T]), bits(wtr["shared"]))
