"""The C++ FfnExec-shaped operator (include/smoe_ffn.hpp, the reference's FfnExec::load / FfnExec::run,
metal/include/strata/metal/layer_exec.hpp:113-140) end to end: stratametal_amd/lib/smoe_ffn_demo loads a
seeded synthetic layer through it, runs one traced call and writes the trace; the same layer and input through
the Python binding must give the same bits (combined output, ids, routing weights, counts)."""
import os
import subprocess
import sys
import tempfile

import numpy as np
import pytest

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
