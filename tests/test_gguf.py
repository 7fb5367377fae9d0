"""GGUF v3 models on the host (smoe_model_*, stratametal_amd/csrc/smoe_gguf.cpp), without a GPU.

- What the reader returns (tensor directory, payload pointers, metadata of every value type) is what the writer in
  tests/gguf_write.py put in the file, for one file and for split models (shard 1 metadata only, as Unsloth's
  splits; the model opened through any shard).
- The reader refuses what the reference's reader refuses (include/strata/artifact/gguf_reader.hpp:420-460,
  500-566; gguf_split.hpp:23-47): a bad magic, another version, a header cut short anywhere, a duplicate tensor
  name, a bad rank, an unknown metadata type, arrays nested too deeply, a data section past the end, a missing
  shard, shard keys that disagree, tensor counts that do not add up, a tensor in two shards, shard 1 opened alone.
  A tensor outside its file or of an unknown type refuses at lookup (GgufModel::in_bounds, tensor_payload_bytes).
- Where oracle/_ref is built, the reference's own GgufModel lists every accepted file identically (shards, data
  offsets, every tensor's name, type, shape, offset, payload bytes and bounds) and refuses every refused one.
- A layer's plan: geometry, types and top_k from the tensors and metadata, 256-byte aligned device slots, and the
  layer refusals (a missing plane, shapes or types that disagree, some hyper-connection tensors only)."""
import ctypes as C
import os

import numpy as np
import pytest

import oracle as O
import stratametal_amd as S
import gguf_write as W


def smoe():
    try:
        return S.lib()
    except ImportError as e:
        pytest.skip(str(e))


def meta_all():
    return [("general.architecture", W.STRING, "qwen4exp"), ("t.u8", W.U8, 250), ("t.i8", W.I8, -3),
            ("t.u16", W.U16, 65000), ("t.i16", W.I16, -300), ("t.u32", W.U32, 4000000000), ("t.i32", W.I32, -7),
            ("t.f32", W.F32, 1.5), ("t.bool", W.BOOL, 1), ("t.str", W.STRING, "héllo"),
            ("t.arr", W.ARRAY, (W.U32, [1, 2, 3, 4, 5])), ("t.sarr", W.ARRAY, (W.STRING, ["a", "bc", ""])),
            ("t.nest", W.ARRAY, (W.ARRAY, [(W.I8, [1, -1]), (W.I8, [])])), ("t.u64", W.U64, 2 ** 63 + 5),
            ("t.i64", W.I64, -(2 ** 40)), ("t.f64", W.F64, -2.25), ("qwen4exp.expert_used_count", W.U32, 4)]


def small_tensors(rng):
    q2 = O.gen_blocks(O.Q2_0, 3, 1, 128 * 3)
    q8 = O.gen_native_blocks(O.Q8_0, 3, 2, 64 * 2)
    q4k = O.gen_native_blocks(O.Q4_K, 3, 3, 256)
    return [W.Tensor("a.f32", (5, 3), W.T_F32, rng.normal(size=15).astype(np.float32)),
            W.Tensor("b.bf16", (7,), W.T_BF16, rng.integers(0, 65535, 7, dtype=np.uint16)),
            W.Tensor("c.q2_0", (128, 3), W.T_Q2_0, q2),
            W.Tensor("d.q8_0", (64, 2), O.Q8_0, q8),
            W.Tensor("e.q4_k", (256, 1, 1, 1), O.Q4_K, q4k)]


def check_model(m: S.Model, want, shard_of=None):
    got = m.tensors()
    assert [t.name for t in got] == [t.name for t in want]
    for g, w in zip(got, want):
        assert g.type == w.type and g.shape == w.ne and g.bytes == len(w.data), g
        assert g.shard == (shard_of[w.name] if shard_of else 0)
        assert m.tensor_bytes(w.name) == w.data
        assert m.tensor(w.name) == g


def test_single_file(tmp_path):
    smoe()
    rng = np.random.default_rng(0)
    ts = small_tensors(rng)
    for align in (32, 64, 1):
        meta = meta_all() + ([("general.alignment", W.U32, align)] if align != 32 else [])
        p = W.write(tmp_path / f"m{align}.gguf", meta, ts, alignment=align)
        m = S.Model(p)
        assert m.n_shards == 1
        check_model(m, ts)
        for t in m.tensors():
            assert t.file_offset % align == 0
        assert m.meta_u64("t.u8") == 250 and m.meta_u64("t.i8") == 2 ** 64 - 3  # signed values sign-extended
        assert m.meta_u64("t.u16") == 65000 and m.meta_u64("t.i16") == 2 ** 64 - 300
        assert m.meta_u64("t.u32") == 4000000000 and m.meta_u64("t.i32") == 2 ** 64 - 7
        assert m.meta_u64("t.bool") == 1 and m.meta_u64("t.u64") == 2 ** 63 + 5 and m.meta_u64("t.i64") == 2 ** 64 - 2 ** 40
        assert m.meta_u64("t.arr") == 5 and m.meta_u64("t.sarr") == 3 and m.meta_u64("t.nest") == 2  # element counts
        assert m.meta_str("t.str") == "héllo" and m.meta_str("general.architecture") == "qwen4exp"
        with pytest.raises(RuntimeError, match="not an integer"):
            m.meta_u64("t.f32")
        with pytest.raises(RuntimeError, match="not a string"):
            m.meta_str("t.u8")
        with pytest.raises(RuntimeError, match="no metadata key"):
            m.meta_u64("t.absent")
        with pytest.raises(RuntimeError, match="no tensor"):
            m.tensor("z")
        m.close()


def test_empty_model_and_tensorless_shard(tmp_path):
    smoe()
    m = S.Model(W.write(tmp_path / "e.gguf", [], []))
    assert m.n_shards == 1 and m.tensors() == []


def test_split_model(tmp_path):
    smoe()
    rng = np.random.default_rng(1)
    ts = small_tensors(rng)
    shards = [[], ts[:2], ts[2:]]  # shard 1: metadata only
    paths = W.write_split(str(tmp_path / "model"), meta_all(), shards)
    shard_of = {t.name: i for i, s in enumerate(shards) for t in s}
    for p in paths:  # any shard opens the whole model
        m = S.Model(p)
        assert m.n_shards == 3
        check_model(m, ts, shard_of)
        assert m.meta_u64("qwen4exp.expert_used_count") == 4  # metadata from shard 1
        m.close()
    # a name that only looks split opens as one file
    q = tmp_path / "model-00001-of-0000x.gguf"
    W.write(q, [], ts[:1])
    assert S.Model(str(q)).n_shards == 1


def bad_files(tmp_path):
    """(name, path, error fragment) of files the reader must refuse at open."""
    rng = np.random.default_rng(2)
    ts = small_tensors(rng)
    out = []

    def one(name, data, frag):
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        out.append((name, str(p), frag))

    good = W.build(meta_all(), ts)
    one("magic", W.build([], ts, magic=b"GGUX"), "magic")
    one("v2", W.build([], ts, version=2), "v2")
    one("v4", W.build([], ts, version=4), "v4")
    one("dup", W.build([], ts + [W.Tensor("c.q2_0", (64,), W.T_Q2_0, ts[2].data[:18])]), "twice")
    raw = bytearray(W.build([], [W.Tensor("r", (4,), W.T_F32, np.zeros(4, np.float32))]))
    i = raw.index(b"r") + 1
    raw[i:i + 4] = (5).to_bytes(4, "little")  # n_dims 5
    one("rank5", bytes(raw), "rank")
    raw[i:i + 4] = (0).to_bytes(4, "little")
    one("rank0", bytes(raw), "rank")
    raw = bytearray(W.build([("k", W.U8, 1)], []))
    raw[raw.index(b"k") + 1:raw.index(b"k") + 5] = (13).to_bytes(4, "little")
    one("metatype", bytes(raw), "metadata value type")
    deep = (W.ARRAY, [(W.ARRAY, [(W.ARRAY, [(W.U8, [1])])])])
    one("nesting", W.build([("deep", W.ARRAY, deep)], []), "nested")
    one("alignstart", W.build([("general.alignment", W.U32, 1 << 20)], []), "past the end")
    one("alignhuge", W.build([("general.alignment", W.U64, 1 << 63)], []), "past the end")
    one("short", b"GGUF\x03\x00", "too short")
    # the header cut short at several places: inside the counts, a key, a value, the tensor directory
    hdr_end = len(W.build(meta_all(), ts)) - sum(len(t.data) for t in ts) - 64
    for cut in (20, 30, 40, 60, 200, hdr_end // 2, hdr_end - 3):
        one(f"cut{cut}", good[:cut], "too short|ends before|past the end")
    return out


def test_refused_files(tmp_path):
    smoe()
    for name, p, frag in bad_files(tmp_path):
        with pytest.raises(RuntimeError, match=frag):
            S.Model(p)


def test_alignment_that_would_wrap_refused(tmp_path):
    """An alignment so large that rounding the data section's start up wraps past 2^64 refuses the file (it
    would otherwise put the data section at the file's start)."""
    smoe()
    p = tmp_path / "wrap.gguf"
    p.write_bytes(W.build([("general.alignment", W.U64, (1 << 64) - 8)], []))
    with pytest.raises(RuntimeError, match="past the end"):
        S.Model(str(p))


def test_every_truncation_refused(tmp_path):
    """Every prefix of a file shorter than its header refuses, none reads past the mapping."""
    smoe()
    ts = small_tensors(np.random.default_rng(3))
    good = W.build(meta_all(), ts)
    m = S.Model(W.write(tmp_path / "g.gguf", meta_all(), ts))
    first = min(t.file_offset for t in m.tensors())
    p = tmp_path / "t.gguf"
    refused = 0
    for n in range(0, first):
        p.write_bytes(good[:n])
        try:
            S.Model(str(p))
        except RuntimeError:
            refused += 1
    # the first tensor sits at the data section's start: every shorter prefix cuts the header or its padding
    assert refused == first


def split_bad(tmp_path):
    ts = small_tensors(np.random.default_rng(4))
    out = []

    def case(name, shards, frag, keys=None, meta=None, drop=None, arch=True):
        stem = str(tmp_path / name)
        m = meta_all() if meta is None else meta
        paths = W.write_split(stem, m if arch else [x for x in m if x[0] != "general.architecture"], shards,
                              keys=keys)
        if not arch:  # rewrite shard 1 without general.architecture
            W.write(paths[0], [x for x in m if x[0] != "general.architecture"] +
                    [("split.count", W.U16, len(shards)), ("split.no", W.U16, 0),
                     ("split.tensors.count", W.I32, sum(len(s) for s in shards))], shards[0])
        if drop is not None:
            os.remove(paths[drop])
        out.append((name, paths[0 if drop != 0 else 1], frag))

    case("missing", [ts[:1], ts[1:3], ts[3:]], "missing", drop=1)
    case("wrongno", [ts[:1], ts[1:]], "shard 2 of 2", keys={1: {"split.no": (W.U16, 0)}})
    case("wrongcount", [ts[:1], ts[1:]], "shard 2 of 2", keys={1: {"split.count": (W.U16, 3)}})
    case("nocount", [ts[:1], ts[1:]], "shard 2 of 2", keys={1: {"split.count": (None, None)}})
    case("tcdisagree", [ts[:1], ts[1:]], "shard 2 of 2", keys={1: {"split.tensors.count": (W.I32, 9)}})
    case("tcsum", [ts[:1], ts[1:]], "split.tensors.count",
         keys={0: {"split.tensors.count": (W.I32, 9)}, 1: {"split.tensors.count": (W.I32, 9)}})
    case("twoshards", [ts[:2], ts[1:]], "two shards")
    case("noarch", [ts[:1], ts[1:]], "general.architecture", arch=False)
    # shard 1 of 2 renamed to a plain name: opened alone
    p = tmp_path / "alone.gguf"
    W.write(p, meta_all() + [("split.count", W.U16, 2), ("split.no", W.U16, 0)], ts)
    out.append(("alone", str(p), "shard 1 of 2"))
    return out


def test_refused_split_models(tmp_path):
    smoe()
    for name, p, frag in split_bad(tmp_path):
        with pytest.raises(RuntimeError, match=frag):
            S.Model(p)


def test_tensor_refusals(tmp_path):
    """Opened, but a tensor past the end of its file, of an unknown type or of rows not whole blocks is refused
    at lookup (the listing too: every listed tensor is one the reader can hand out)."""
    smoe()
    f = np.zeros(16, np.float32)
    for ts, name, frag in (([W.Tensor("p", (16,), W.T_F32, f), W.Tensor("q", (16,), W.T_F32, f, offset=1 << 20)], "q",
                            "does not fit"),
                           ([W.Tensor("u", (32,), 31, np.zeros(64, np.uint8))], "u", "no known block size"),
                           ([W.Tensor("r", (33,), O.Q8_0, np.zeros(34, np.uint8))], "r", "no known block size"),
                           ([W.Tensor("o", (2 ** 62, 8), W.T_F32, f)], "o", "no known block size")):
        p = W.write(tmp_path / f"{name}.gguf", [], ts)
        m = S.Model(p)
        with pytest.raises(RuntimeError, match=frag):
            m.tensor(name)
        with pytest.raises(RuntimeError, match=frag):
            m.tensors()


def test_model_handle_refusals():
    L = smoe()
    h = C.c_void_p()
    assert L.smoe_model_open(None, C.byref(h)) == -6
    assert L.smoe_model_open(b"/nonexistent/x.gguf", C.byref(h)) == -1 and not h.value
    assert L.smoe_model_n_shards(None) == 0 and L.smoe_model_n_tensors(None) == 0
    L.smoe_model_close(None)


# ---- the reference's reader on the same files ----

def test_reference_reader_agrees(tmp_path):
    smoe()
    if O.ref() is None:
        pytest.skip("oracle/_ref absent (no /root/reference here): the reader is pinned by the writer's files")
    rng = np.random.default_rng(5)
    ts = small_tensors(rng)
    files = [W.write(tmp_path / "one.gguf", meta_all(), ts),
             W.write(tmp_path / "al.gguf", meta_all() + [("general.alignment", W.U32, 128)], ts, alignment=128),
             W.write(tmp_path / "empty.gguf", [], [])]
    files += W.write_split(str(tmp_path / "sp"), meta_all(), [[], ts[:2], ts[2:]])[1:2]
    refused = [p for _, p, _ in bad_files(tmp_path)] + [p for _, p, _ in split_bad(tmp_path)]
    for p in files:
        rc, text = O.ref_gguf_list(p)
        assert rc == 0, text
        m = S.Model(p)
        got = m.tensors()
        want = []
        shard_start = {}
        for line in text.strip().split("\n"):
            f = line.split()
            if f[0] == "shard":
                shard_start[int(f[1])] = int(f[2])
                cur = int(f[1])
                continue
            nd = int(f[2])
            want.append((f[0], int(f[1]), tuple(int(x) for x in f[3:3 + nd]), cur,
                         shard_start[cur] + int(f[3 + nd]), int(f[4 + nd]), f[5 + nd]))
        assert m.n_shards == len(shard_start)
        assert [(t.name, t.type, t.shape, t.shard, t.file_offset, t.bytes, "1") for t in got] == want, p
    for p in refused:
        rc, text = O.ref_gguf_list(p)
        assert rc == -1, (p, text)
        with pytest.raises(RuntimeError):
            S.Model(p)
    # tensors the reference reader lists as out of bounds are the ones this reader refuses at lookup
    f = np.zeros(16, np.float32)
    p = W.write(tmp_path / "oob.gguf", [], [W.Tensor("p", (16,), W.T_F32, f), W.Tensor("q", (16,), W.T_F32, f,
                                                                                    offset=1 << 20)])
    rc, text = O.ref_gguf_list(p)
    flags = {ln.split()[0]: ln.split()[-1] for ln in text.strip().split("\n") if not ln.startswith("shard")}
    assert flags == {"p": "1", "q": "0"}
    m = S.Model(p)
    assert m.tensor("p").bytes == 64
    with pytest.raises(RuntimeError):
        m.tensor("q")


# ---- a layer's plan ----

def small_geom(**kw):
    d = dict(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=8, top_k=2)
    d.update(kw)
    return O.Geom(**d)


def hc_arrays(H, n=4, lr=8, seed=0):
    rng = np.random.default_rng(seed)
    return (n, lr, (1 + rng.normal(size=n * H) * 0.1).astype(np.float32),
            W.bf16_rne(rng.normal(size=lr * n * H) * 0.05), W.bf16_rne(rng.normal(size=n * H * lr) * 0.05),
            W.bf16_rne(rng.normal(size=n * n * H) * 0.05))


@pytest.mark.parametrize("case", ["q2_0", "iq2_s", "native_shared", "f32_router", "no_shared", "hc"])
def test_layer_plan(tmp_path, case):
    smoe()
    if case == "iq2_s":
        g = small_geom(n_embd=512, n_ff=512, n_ff_shared=512, w_type=O.IQ2_S, sh_type=O.IQ2_S)
    elif case == "native_shared":
        g = small_geom(sh_type=O.Q4_K, sh_up_type=O.Q5_0, sh_down_type=O.Q6_K, n_ff_shared=256)
    elif case == "f32_router":
        g = small_geom(router_dtype=1)
    elif case == "no_shared":
        g = small_geom(sh_type=-1)
    else:
        g = small_geom()
    w = O.make_weights(g, 11)
    hc = hc_arrays(g.n_embd) if case == "hc" else None
    ts = W.layer_tensors(g, w, 3, hc=hc) + W.layer_tensors(g, w, 4)
    p = W.write(tmp_path / "layer.gguf", [("general.architecture", W.STRING, "qwen4exp"),
                                         ("qwen4exp.expert_used_count", W.U32, g.top_k)], ts)
    m = S.Model(p)
    pl = m.plan(3, with_shared=g.sh_type >= 0)
    gc = pl.geom
    assert (gc.n_embd, gc.n_ff, gc.n_expert, gc.top_k, gc.w_type, gc.router_dtype) == \
        (g.n_embd, g.n_ff, g.n_expert, g.top_k, g.w_type, g.router_dtype)
    if g.sh_type >= 0:
        assert (gc.n_ff_shared, gc.sh_gate_type, gc.sh_up_type, gc.sh_down_type) == (g.n_ff_shared,) + g.shared_types()
    else:
        assert gc.sh_type == -1
    assert (pl.hc.hc, pl.hc.hc_lr) == ((4, 8) if hc else (0, 0))
    offs = [pl.off[i] for i in range(12)]
    used = [0, 1, 2, 3] + ([4, 5, 6, 7] if g.sh_type >= 0 else []) + ([8, 9, 10, 11] if hc else [])
    sizes = {0: w.gate_exps.nbytes, 1: w.up_exps.nbytes, 2: w.down_exps.nbytes, 3: w.router.nbytes}
    if g.sh_type >= 0:
        sizes.update({4: w.gate_sh.nbytes, 5: w.up_sh.nbytes, 6: w.down_sh.nbytes, 7: g.n_embd * 2})
    if hc:
        sizes.update({8: hc[2].nbytes, 9: hc[3].nbytes, 10: hc[4].nbytes, 11: hc[5].nbytes})
    end = 0
    for i in used:  # in order, 256-byte aligned, each slot its tensor's bytes
        assert offs[i] % 256 == 0 and offs[i] >= end
        end = offs[i] + sizes[i]
    assert pl.device_bytes >= end and pl.device_bytes - end < 256
    assert m.plan(3, top_k=1, with_shared=False).geom.top_k == 1
    assert m.plan(4, with_shared=g.sh_type >= 0).hc.hc == 0


def test_layer_plan_refusals(tmp_path):
    smoe()
    g = small_geom()
    w = O.make_weights(g, 12)
    arch = [("general.architecture", W.STRING, "qwen4exp")]

    def model(ts, meta=arch):
        p = tmp_path / f"l{len(os.listdir(tmp_path))}.gguf"
        return S.Model(W.write(p, meta, ts))

    full = W.layer_tensors(g, w, 0, hc=hc_arrays(g.n_embd))
    with pytest.raises(RuntimeError, match="expert_used_count"):  # no top_k and none declared
        model(full).plan(0)
    for drop, frag in (("blk.0.ffn_up_exps.weight", "has no blk.0.ffn_up_exps"),
                       ("blk.0.ffn_gate_inp.weight", "has no"), ("blk.0.ffn_down_shexp.weight", "has no"),
                       ("blk.0.hc_ffn_up.weight", "only some of the hc_ffn")):
        m = model([t for t in full if t.name != drop])
        with pytest.raises(RuntimeError, match=frag):
            m.plan(0, top_k=2)
    assert model([t for t in full if "shexp" not in t.name]).plan(0, top_k=2, with_shared=False).geom.sh_type == -1
    with pytest.raises(RuntimeError, match="has no"):
        model(full).plan(1, top_k=2)

    def swap(name, **kw):
        out = []
        for t in full:
            if t.name == name:
                t = W.Tensor(t.name, kw.get("ne", t.ne), kw.get("type_", t.type), kw.get("data", t.data))
            out.append(t)
        return out

    H, F, E = g.n_embd, g.n_ff, g.n_expert
    for ts, frag in ((swap("blk.0.ffn_up_exps.weight", ne=(H, F // 2, E * 2)), "shape"),
                     (swap("blk.0.ffn_down_exps.weight", ne=(H, F, E)), "shape"),
                     (swap("blk.0.ffn_gate_inp.weight", ne=(H, E + 1), data=w.router.tobytes() + b"\0" * H * 2),
                      "shape"),
                     (swap("blk.0.ffn_gate_inp.weight", type_=W.T_F16), "neither BF16 nor F32"),
                     (swap("blk.0.ffn_up_exps.weight", type_=W.T_IQ2_S, data=w.up_exps.tobytes()[:E * F * H // 256 * 82]),
                      "different types"),
                     (swap("blk.0.ffn_gate_inp_shexp.weight", ne=(H, 2), data=w.gate_inp_sh.tobytes() * 2),
                      "not \\[n_embd\\]"),
                     (swap("blk.0.hc_ffn_inject.weight", type_=W.T_F32,
                           data=np.zeros(4 * 4 * H, np.float32)), "must be BF16"),
                     (swap("blk.0.hc_ffn_norm.weight", ne=(4 * H - 1,), data=np.zeros(4 * H - 1, np.float32)),
                      "disagree"),
                     (swap("blk.0.hc_ffn_inject.weight", ne=(65 * H, 65), data=np.zeros(65 * 65 * H, np.uint16)),
                      "implausible hc_ffn")):
        with pytest.raises(RuntimeError, match=frag):
            model(ts).plan(0, top_k=2)
    # a geometry the block does not run: the library's own reason
    with pytest.raises(RuntimeError, match="top_k"):
        model(full).plan(0, top_k=9)
    # a shared projection of a type the block does not run: an F32 (GGML type 0) or F16 plane is refused, never read
    # as the shared expert's own type (a zero type in smoe_geom means "as sh_type")
    Fs = g.n_ff_shared
    for name, ne in (("blk.0.ffn_down_shexp.weight", (Fs, H)), ("blk.0.ffn_up_shexp.weight", (H, Fs))):
        for t in (W.T_F32, W.T_F16):
            data = np.zeros(Fs * H, np.float32 if t == W.T_F32 else np.float16)
            with pytest.raises(RuntimeError, match=f"GGML type {t}"):
                model(swap(name, type_=t, data=data)).plan(0, top_k=2)
    # a dimension beyond int32 (it would narrow to a geometry the block accepts) and a top_k beyond 64 are refused
    # (the plane's 1.2 GB payload is a hole of a sparse file: nothing is written and nothing is read)
    big = [W.Tensor(t.name, (2 ** 32 + H, 1, 1), t.type, b"", offset=0) if t.name == "blk.0.ffn_gate_exps.weight"
           else t for t in full]
    pbig = W.write(tmp_path / "big.gguf", arch, big)
    os.truncate(pbig, os.path.getsize(pbig) + (2 ** 32 + H) // 64 * 18)
    with pytest.raises(RuntimeError, match="beyond int32"):
        S.Model(pbig).plan(0, top_k=2)
    with pytest.raises(RuntimeError, match="beyond 64"):
        model(full, arch + [("qwen4exp.expert_used_count", W.U64, 2 ** 32 + 2)]).plan(0)


def test_repeated_metadata_key_keeps_the_first(tmp_path):
    """A key listed twice keeps its first value, as the reference reader's map (emplace) does."""
    smoe()
    g = small_geom()
    w = O.make_weights(g, 13)
    meta = [("general.architecture", W.STRING, "qwen4exp"), ("qwen4exp.expert_used_count", W.U32, 2),
            ("qwen4exp.expert_used_count", W.U32, 3)]
    m = S.Model(W.write(tmp_path / "dup.gguf", meta, W.layer_tensors(g, w, 0)))
    assert m.plan(0).geom.top_k == 2
