"""GGUF layers loaded into device memory (smoe_layer_plan_for / smoe_layer_upload through stratametal_amd.Model)
and run: the loaded bytes are the file's, and the block on them gives the oracle's bits on the same host arrays.

The files are written by tests/gguf_write.py from the oracle's generators (the layout FfnExec::load reads,
metal/src/layer_exec.cpp:369-431): routed Q2_0 and IQ2_S planes, BF16 and F32 routers, the shared expert in the
routed type and in its own native types with a BF16 or an F32 gate (uploaded as bf16, round to nearest even), the
hyper-connection tensors, one file and a split model."""
import sys

import numpy as np
import pytest

import oracle as O
import stratametal_amd as S
import gguf_write as W

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


def hc_arrays(H, n=4, lr=8, seed=0):
    rng = np.random.default_rng(seed)
    return (n, lr, (1 + rng.normal(size=n * H) * 0.1).astype(np.float32),
            W.bf16_rne(rng.normal(size=lr * n * H) * 0.05), W.bf16_rne(rng.normal(size=n * H * lr) * 0.05),
            W.bf16_rne(rng.normal(size=n * n * H) * 0.05))


CASES = [
    # name, geometry, seed, tokens, split shards, F32 shared gate, hc tensors
    ("Q2_0 routed and shared, BF16 router, hc tensors", dict(n_expert=64, top_k=8), 81, (1, 16), 1, False, True),
    ("IQ2_S routed, Q8_0 shared, split in 3", dict(n_embd=512, n_ff=512, n_ff_shared=512, n_expert=16, top_k=4,
                                                  w_type=O.IQ2_S, sh_type=O.Q8_0), 82, (1, 5), 3, False, False),
    ("Q2_0 routed, Q3_K/IQ4_NL shared, F32 router and shared gate",
     dict(n_expert=32, top_k=4, router_dtype=1, sh_type=O.Q3_K, sh_down_type=O.IQ4_NL), 83, (2, 40), 2, True, False),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_gguf_layer_forward(torch, tmp_path, case):
    name, gkw, seed, tokens, n_split, f32_gate, with_hc = CASES[case]
    say(f"case: gguf layer {name}")
    g = O.Geom(**gkw)
    w = O.make_weights(g, seed)
    gate_inp = None
    if f32_gate:  # stored F32; the block's contract takes it as bf16, rounded to nearest even on upload
        v = (np.random.default_rng(seed).normal(size=g.n_embd) * 0.3).astype(np.float32)
        gate_inp = (W.T_F32, v)
        w.gate_inp_sh = W.bf16_rne(v)
    hc = hc_arrays(g.n_embd, seed=seed) if with_hc else None
    layer = 5
    ts = W.layer_tensors(g, w, layer, gate_inp_sh=gate_inp, hc=hc) + W.layer_tensors(g, w, layer + 1)
    meta = [("general.architecture", W.STRING, "qwen4exp"), ("qwen4exp.expert_used_count", W.U32, g.top_k)]
    if n_split == 1:
        path = W.write(tmp_path / "m.gguf", meta, ts)
    else:
        per = -(-len(ts) // (n_split - 1))
        shards = [[]] + [ts[i * per:(i + 1) * per] for i in range(n_split - 1)]
        path = W.write_split(str(tmp_path / "m"), meta[1:], shards, arch="qwen4exp")[-1]
    m = S.Model(path)
    assert m.n_shards == n_split
    gl, wd, hcx = m.load_layer(layer, with_hc=with_hc)
    assert (gl.n_embd, gl.n_ff, gl.n_expert, gl.top_k, gl.w_type, gl.router_dtype) == \
        (g.n_embd, g.n_ff, g.n_expert, g.top_k, g.w_type, g.router_dtype)
    # the device bytes are the file's (the F32 shared gate as its bf16 rounding)
    for k in ("gate_exps", "up_exps", "down_exps", "router", "gate_sh", "up_sh", "down_sh", "gate_inp_sh"):
        want = getattr(w, k)
        assert host(torch, wd[k]).tobytes() == np.ascontiguousarray(want).tobytes(), k
    if with_hc:
        for t, a in zip(hcx.tensors, hc[2:]):
            assert host(torch, t).tobytes() == a.tobytes()
        assert (hcx.hc, hcx.hc_lr) == hc[:2]
    ml = S.MoELayer(gl, wd, max_tokens=max(tokens))
    for T in tokens:
        say(f"case: gguf layer {name} T={T}")
        x = O.gen_normal(seed, 100 + T, T * g.n_embd).reshape(T, g.n_embd)
        y = ml.forward(dev(torch, x))
        want = O.moe_decode_dev(g, w, x, n_threads=8)
        assert np.array_equal(bits(host(torch, y)), bits(want)), f"T={T} max rel {O.rel_l1_rows(host(torch, y), want).max()}"
    m.close()  # the device copy stays valid without the mapping
    x = O.gen_normal(seed, 99, g.n_embd).reshape(1, g.n_embd)
    assert np.array_equal(bits(host(torch, ml.forward(dev(torch, x)))), bits(O.moe_decode_dev(g, w, x, n_threads=8)))


def test_gguf_upload_refusals(torch, tmp_path):
    say("case: gguf upload refusals")
    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=8, top_k=2)
    w = O.make_weights(g, 3)
    m = S.Model(W.write(tmp_path / "r.gguf", [], W.layer_tensors(g, w, 0) + W.layer_tensors(g, w, 1)))
    p = m.plan(0, top_k=2)
    L = S.lib()
    buf = torch.zeros(p.device_bytes + 512, dtype=torch.uint8, device="cuda")
    base = (buf.data_ptr() + 255) & ~255
    wc, hc = S._Weights(), S._Hc()
    st = S._stream(None)
    import ctypes as C
    assert L.smoe_layer_upload(m._h, C.byref(p), base + 16, p.device_bytes, C.byref(wc), None, st) == -5
    assert L.smoe_layer_upload(m._h, C.byref(p), base, p.device_bytes - 1, C.byref(wc), None, st) == -2
    assert L.smoe_layer_upload(m._h, C.byref(p), base, p.device_bytes, C.byref(wc), C.byref(hc), st) == -1
    p1 = m.plan(1, top_k=2)
    p1.layer = 0  # another layer's plan presented as layer 0's: same slots here, so give it other slots
    p1.off[1] += 256
    assert L.smoe_layer_upload(m._h, C.byref(p1), base, p.device_bytes, C.byref(wc), None, st) == -1
    assert not host(torch, buf).any(), "a refused upload wrote"
    assert L.smoe_layer_upload(m._h, C.byref(p), base, p.device_bytes, C.byref(wc), None, st) == 0
    assert host(torch, buf).any()


def _demo_out(raw, T, H, E, K, n_layer):
    hdr = np.frombuffer(raw[:16], np.int32)
    assert list(hdr) == [T, H, E, K]
    o = 16
    parts = []
    for dtype, n in ((np.float32, T * H), (np.int32, T * K), (np.float32, T * K), (np.int32, E), (np.float32, 5),
                     (np.float32, n_layer)):
        parts.append(np.frombuffer(raw[o:o + 4 * n], dtype))
        o += 4 * n
    assert o == len(raw)
    return parts


def test_cpp_operator_loads_a_gguf_layer(torch, tmp_path):
    """The C++ operator's load(model, layer, geometry, with_shared) (FfnExec::load, metal/src/layer_exec.cpp:
    369-452) on a GGUF layer with hyper-connection tensors: its traced run and its layer call give the bits of the
    Python binding on the same file and inputs; a geometry the layer does not have is refused."""
    import os
    import subprocess
    demo = os.path.join(os.path.dirname(S.LIB_PATH), "smoe_ffn_demo")
    assert os.path.exists(demo), "smoe_ffn_demo is not built (python -m stratametal_amd.build)"
    g = O.Geom(n_expert=64, top_k=8)
    seed, layer, T = 84, 3, 7
    say(f"case: C++ FfnExec::load from GGUF, T={T}")
    w = O.make_weights(g, seed)
    hc = hc_arrays(g.n_embd, seed=seed)
    ts = W.layer_tensors(g, w, layer, hc=hc) + W.layer_tensors(g, w, layer + 1)
    meta = [("general.architecture", W.STRING, "qwen4exp"), ("qwen4exp.expert_used_count", W.U32, g.top_k)]
    path = str(W.write(tmp_path / "m.gguf", meta, ts))
    out = str(tmp_path / "out.bin")
    H, E, K, n_hc, lr = g.n_embd, g.n_expert, g.top_k, hc[0], hc[1]
    args = [demo, "--gguf", out, path, str(layer), str(T), str(seed), str(H), str(g.n_ff), str(E), str(n_hc),
            str(lr), "1"]
    r = subprocess.run(args, capture_output=True, text=True, timeout=120)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stderr
    comb, ids, rw, counts, stage_ms, lay = _demo_out(open(out, "rb").read(), T, H, E, K, T * n_hc * H)
    assert (stage_ms >= 0).all()

    m = S.Model(path)
    gl, wd, hcx = m.load_layer(layer, with_hc=True)
    x = S.synth_normal(seed, 100, T * H).reshape(T, H)
    ml = S.MoELayer(gl, wd, max_tokens=T)
    y, tr = ml.forward(x, add_shared=True, trace=True)
    assert np.array_equal(comb.view(np.uint32), bits(host(torch, y)).ravel())
    assert np.array_equal(ids, host(torch, tr["ids"]).ravel())
    assert np.array_equal(rw.view(np.uint32), bits(host(torch, tr["weights"])).ravel())
    assert np.array_equal(counts, host(torch, tr["counts"]))
    # the oracle's bits on the file's arrays, as the forward test above checks them
    assert np.array_equal(comb.view(np.uint32), bits(O.moe_decode_dev(g, w, host(torch, x), n_threads=8)).ravel())
    R = S.synth_normal(seed, 101, T * n_hc * H).reshape(T, n_hc, H)
    got = S.FfnLayer(gl, wd, hcx, max_tokens=T).run(R)
    assert np.array_equal(lay.view(np.uint32), bits(host(torch, got)).ravel())
    m.close()

    bad = list(args)
    bad[8] = str(2 * g.n_ff)  # n_ff the layer does not have
    r = subprocess.run(bad, capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "the geometry says" in r.stderr, (r.returncode, r.stderr)
