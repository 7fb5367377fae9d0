"""The C++ FfnExec-shaped operator (include/smoe_ffn.hpp, the reference's FfnExec::load / FfnExec::run,
metal/include/strata/metal/layer_exec.hpp:113-140) end to end: stratametal_amd/lib/smoe_ffn_demo loads a
seeded synthetic layer through it, runs one traced call and writes the trace, then the whole layer call with the
hyper-connection ends (FfnExec::run_layer); the same layer and inputs through the Python binding must give the same
bits (combined output, ids, routing weights, counts, the layer's residual streams)."""
import os
import subprocess
import sys
import tempfile

import numpy as np
import pytest

import oracle as O

import stratametal_amd as S

pytestmark = pytest.mark.gpu
DEMO = os.path.join(os.path.dirname(S.LIB_PATH), "smoe_ffn_demo")


@pytest.fixture(scope="module")
def torch():
    import torch as T
    if not T.cuda.is_available():
        pytest.skip("no GPU")
    S.lib()
    return T


@pytest.mark.parametrize("T,seed,geom", [(5, 11, (256, 128, 128, 16, 4)), (16, 2, (2048, 512, 512, 512, 10))])
def test_cpp_operator_matches_python_binding(torch, T, seed, geom):
    print(f"case: C++ FfnExec T={T} geom={geom}", flush=True)
    assert os.path.exists(DEMO), "smoe_ffn_demo is not built (python -m stratametal_amd.build)"
    H, F, Fs, E, K = geom
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "trace.bin")
        r = subprocess.run([DEMO, out, str(T), str(seed), *map(str, geom)], capture_output=True, text=True,
                           timeout=120)
        sys.stdout.write(r.stdout)
        assert r.returncode == 0, r.stderr
        raw = open(out, "rb").read()
    hdr = np.frombuffer(raw[:16], np.int32)
    assert list(hdr) == [T, H, E, K]
    o = 16
    def take(dtype, n):
        nonlocal o
        a = np.frombuffer(raw[o:o + 4 * n], dtype)
        o += 4 * n
        return a
    comb = take(np.float32, T * H).reshape(T, H)
    ids = take(np.int32, T * K).reshape(T, K)
    rw = take(np.float32, T * K).reshape(T, K)
    counts = take(np.int32, E)
    stage_ms = take(np.float32, 5)
    layer_out = take(np.float32, T * 4 * H).reshape(T, 4, H)
    assert o == len(raw) and (stage_ms >= 0).all()

    g = S.Geom(n_embd=H, n_ff=F, n_ff_shared=Fs, n_expert=E, top_k=K)
    w = S.synth_layer(g, seed)
    x = S.synth_normal(seed, 100, T * H).reshape(T, H)
    ml = S.MoELayer(g, w, max_tokens=T)
    y, tr = ml.forward(x, add_shared=True, trace=True)
    torch.cuda.synchronize()
    assert np.array_equal(comb.view(np.uint32), y.cpu().numpy().view(np.uint32))
    assert np.array_equal(ids, tr["ids"].cpu().numpy().reshape(T, K))
    assert np.array_equal(rw.view(np.uint32), tr["weights"].cpu().numpy().reshape(T, K).view(np.uint32))
    assert np.array_equal(counts, tr["counts"].cpu().numpy())
    # the layer call: the same hyper-connection tensors (the oracle's generators equal the device ones bitwise)
    hw = O.make_hc(H, 4, 320, seed)
    up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    hcd = S.HyperConnection(H, 4, 320, up(hw.norm), up(hw.down.view(np.int16)), up(hw.up.view(np.int16)),
                            up(hw.inject.view(np.int16)), eps=1e-6)
    R = S.synth_normal(seed, 101, T * 4 * H).reshape(T, 4, H)
    got = S.FfnLayer(g, w, hcd, max_tokens=T).run(R)
    torch.cuda.synchronize()
    assert np.array_equal(layer_out.view(np.uint32), got.cpu().numpy().view(np.uint32))
