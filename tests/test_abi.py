"""CPU tests of the C ABI: libsmoe.so loads, exports every function include/smoe.h declares, and refuses bad
arguments (or accepts zero counts) before any HIP call, so these run without a GPU.  The pointers passed are
never dereferenced: every case below returns during argument checking (metal/src/router_parity.cpp:195-225,
metal/src/moe_combine_parity.cpp refusal cases)."""
import ctypes as C
import os
import re
import subprocess

import pytest

import stratametal_amd as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = 0x10000000  # a 256-byte aligned address that is never dereferenced by a refused / empty call


def declared_functions():
    text = open(os.path.join(ROOT, "include", "smoe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(smoe_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = S.lib()
    names = declared_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", S.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (smoe_\w+)", out))
    assert set(names) <= exported


def test_abi_version_and_status_strings():
    lib = S.lib()
    assert lib.smoe_abi_version() == 109
    for code in (0, -1, -2, -3, -4, -5, -6):
        assert lib.smoe_status_str(code)


def _ws(g):
    return S.lib().smoe_workspace_bytes(C.byref(g.c()), 16)


def test_workspace_size_and_geometry_refusals():
    assert _ws(S.Geom()) > 0
    assert _ws(S.Geom(router_dtype=1)) > 0  # the f32 router
    bad = [S.Geom(top_k=65), S.Geom(n_expert=1025), S.Geom(top_k=20, n_expert=10), S.Geom(n_embd=2000),
           S.Geom(n_ff=100), S.Geom(w_type=13), S.Geom(router_dtype=2), S.Geom(router_dtype=-1), S.Geom(n_embd=8192)]
    for g in bad:
        assert _ws(g) == 0, g


def _forward(g, T, ws_bytes=1 << 30, path=0, weights=None, add_shared=1):
    L = S.lib()
    w = weights if weights is not None else S._Weights(*([FAKE] * 8 + [None]))
    return L.smoe_forward_path(C.byref(g.c()), C.byref(w), FAKE, T, FAKE, add_shared, FAKE, ws_bytes, None, path,
                               None)


def test_forward_refusals_before_launch():
    g = S.Geom()
    assert _forward(S.Geom(top_k=65), 1) == -1
    assert _forward(S.Geom(n_expert=2048), 1) == -1
    assert _forward(S.Geom(w_type=7), 1) == -3
    assert _forward(g, -1) == -1
    assert _forward(g, 1, path=9) == -1
    assert _forward(g, 1, ws_bytes=1024) == -2
    assert "needs" in S.lib().smoe_last_error().decode()
    null_router = S._Weights(FAKE, FAKE, FAKE, None, FAKE, FAKE, FAKE, FAKE, None)
    assert _forward(g, 1, weights=null_router) == -6
    misaligned = S._Weights(FAKE + 2, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None)
    assert _forward(g, 1, weights=misaligned) == -5
    # launch grids hold at most 65535 tokens or work items on their y dimension: refused before the first launch
    small = S.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=64, top_k=64)
    assert _forward(small, 65536, path=2) == -1
    assert "split the batch" in S.lib().smoe_last_error().decode()
    assert _forward(small, 65536, path=1) == -1


def test_forward_zero_tokens_returns_ok_without_launching():
    assert _forward(S.Geom(), 0) == 0


def test_forward_residual_refusals_before_launch():
    """The fused stack junction refuses an x that overlaps x_prev, r_prev or y, a NULL r_prev and misaligned rows
    before any launch; zero tokens return at once."""
    L, g = S.lib(), S.Geom()
    w = S._Weights(*([FAKE] * 8 + [None]))
    R, X, Y = FAKE + (1 << 24), FAKE + (2 << 24), FAKE + (3 << 24)

    def call(xp, rp, x, y, T=1):
        return L.smoe_forward_residual(C.byref(g.c()), C.byref(w), xp, rp, 1e-6, x, T, y, 1, FAKE, 1 << 30, None,
                                       None)

    assert call(FAKE, R, X, Y, T=0) == 0
    assert call(FAKE, R, FAKE, Y) == -1
    assert call(FAKE, R, R + 256, Y) == -1
    assert call(FAKE, R, X, X) == -1
    assert call(FAKE, None, X, Y) == -6
    assert call(None, R, X, Y) == -6
    assert call(FAKE, R, X + 4, Y) == -5


def test_stage_refusals_and_zero_counts():
    L = S.lib()
    # router: k = 65, 1025 experts, a negative count, k above n_expert (metal/src/router_parity.cpp:195-218)
    assert L.smoe_router_topk(FAKE, 1, 128, 65, FAKE, FAKE, None) == -1
    assert L.smoe_router_topk(FAKE, 1, 1025, 1, FAKE, FAKE, None) == -1
    assert L.smoe_router_topk(FAKE, -1, 32, 4, FAKE, FAKE, None) == -1
    assert L.smoe_router_topk(FAKE, 1, 4, 8, FAKE, FAKE, None) == -1
    assert L.smoe_router_topk(FAKE, 0, 512, 10, FAKE, FAKE, None) == 0       # zero tokens: no launch
    assert L.smoe_router_margin(FAKE, 1, 10, 10, FAKE, FAKE, None) == -1     # needs k < n_expert
    assert L.smoe_router_margin(FAKE, 1, 1025, 10, FAKE, FAKE, None) == -1
    assert L.smoe_router_margin(FAKE, 1, 512, 0, FAKE, FAKE, None) == -1
    assert L.smoe_router_margin(None, 1, 512, 10, FAKE, FAKE, None) == -6
    assert L.smoe_router_margin(FAKE + 2, 1, 512, 10, FAKE, FAKE, None) == -5
    assert L.smoe_router_margin(FAKE, 0, 512, 10, FAKE, FAKE, None) == 0     # zero tokens: no launch
    # combine: k = 65, negative, zero (metal/src/moe_combine_parity.cpp)
    assert L.smoe_combine(FAKE, FAKE, None, FAKE, 16, 65, None) == -1
    assert L.smoe_combine(FAKE, FAKE, None, FAKE, -1, 4, None) == -1
    assert L.smoe_combine(FAKE, FAKE, None, FAKE, 0, 10, None) == 0
    assert L.smoe_combine(FAKE, FAKE, None, FAKE, 256, 0, None) == 0
    # q8_1 / swiglu: lengths that are not whole blocks
    assert L.smoe_quantize_q8_1(FAKE, 33, FAKE, None) == -1
    assert L.smoe_swiglu_q8(FAKE, FAKE, 40, FAKE, None) == -1
    assert L.smoe_quantize_q8_1(FAKE, 0, FAKE, None) == 0
    # mmvq: a type that is not built, a length that is not whole double blocks
    assert L.smoe_mmvq(29, FAKE, 0, FAKE, 256, 4, 1, FAKE, None) == -3
    assert L.smoe_mmvq(42, FAKE, 0, FAKE, 192, 4, 1, FAKE, None) == -1
    assert L.smoe_mmvq(42, FAKE, 2, FAKE, 256, 4, 1, FAKE, None) == -5
    assert L.smoe_mmvq(42, FAKE, 0, FAKE, 256, 0, 1, FAKE, None) == 0
    # dispatch
    assert L.smoe_dispatch(FAKE, 4, 10, 2000, FAKE, FAKE, FAKE, FAKE, None) == -1
    assert L.smoe_dispatch(FAKE, 0, 10, 512, FAKE, FAKE, FAKE, FAKE, None) == 0
    # synthetic generators
    assert L.smoe_synth_blocks(42, 1, 1, 100, 0.02, FAKE, None) == -1
    assert L.smoe_synth_blocks(5, 1, 1, 64, 0.02, FAKE, None) == -3


def test_product_has_no_oracle_dependency():
    """The product never imports, links or loads the test oracle (its CPU restatement)."""
    pkg = os.path.join(ROOT, "stratametal_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(import|from)\s+oracle\b", text, re.M), f
                assert not re.search(r'#include\s*[<"][^>"]*smoe_oracle', text), f
                assert "liboracle" not in text, f
    out = subprocess.run(["ldd", S.LIB_PATH], capture_output=True, text=True).stdout
    assert "oracle" not in out


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(S, "_LIB", None)
    monkeypatch.setattr(S, "LIB_PATH", "/nonexistent/libsmoe.so")
    with pytest.raises(ImportError):
        S.lib()


def test_expert_sizes_and_refusals():
    L = S.lib()
    # the reference's iq_expert_bytes: 2 * n_ff * gate row + n_embd * down row (metal/src/iq.mm:171-180)
    assert L.smoe_expert_bytes(S.IQ2_S, S.Q2_0, 2048, 512) == 2 * 512 * (2048 // 256 * 82) + 2048 * (512 // 64 * 18)
    assert L.smoe_expert_bytes(S.IQ2_S, S.IQ2_S, 2048, 512) == 2 * 512 * 656 + 2048 * (512 // 256 * 82)
    assert L.smoe_expert_bytes(S.Q2_0, S.Q2_0, 2048, 512) == 0
    assert b"down quant" in L.smoe_last_error()
    assert L.smoe_expert_bytes(S.IQ2_S, S.Q2_0, 2048, 0) == 0
    assert L.smoe_expert_bytes(S.IQ2_S, 13, 2048, 512) == 0
    need = L.smoe_expert_bytes(S.IQ2_S, S.Q2_0, 2048, 512)
    sc = L.smoe_expert_scratch_bytes(2048, 512, 4)
    args = lambda blob_bytes, gu, n_tok, sc_bytes: (FAKE, blob_bytes, FAKE, gu, S.Q2_0, 2048, 512, n_tok, FAKE, FAKE,
                                                    sc_bytes, None)
    assert L.smoe_expert(*args(need, S.IQ2_S, 0, 0)) == 0          # zero tokens: nothing to do
    assert L.smoe_expert(*args(need, S.IQ2_S, -1, sc)) == -1       # negative count
    assert L.smoe_expert(*args(need, S.Q2_0, 4, sc)) == -3         # a 64-value gate type
    assert L.smoe_expert(*args(need - 1, S.IQ2_S, 4, sc)) == -2    # blob too small
    assert f"expert blob is {need - 1} bytes, needs {need}".encode() in L.smoe_last_error()
    assert L.smoe_expert(*args(need, S.IQ2_S, 4, sc - 1)) == -2    # scratch too small


def test_forward_static_refusals_before_launch():
    """The no-allocation entry point refuses a batch whose workspace exceeds the static scratch (with the limit in
    the message) and bad geometry before any HIP call; zero tokens return at once."""
    L, g = S.lib(), S.Geom()
    w = S._Weights(*([FAKE] * 8 + [None]))

    def call(gg, T):
        return L.smoe_forward_static(C.byref(gg.c()), C.byref(w), FAKE, T, FAKE, 1, None, None)

    assert call(g, 0) == 0
    assert call(g, -1) == -1
    assert call(S.Geom(top_k=65), 1) == -1
    limit = 32 << 20
    T = next(t for t in range(1, 4096) if L.smoe_workspace_bytes(C.byref(g.c()), t) > limit)
    assert T > 128  # covers every decode batch and the smallest prefill batches of the benchmark geometry
    assert call(g, T) == -2
    assert str(limit).encode() in L.smoe_last_error()


def test_binding_refuses_bad_tensors_before_launch():
    """The Python binding checks dtype, contiguity, shape and device before any ctypes call (a wrong tensor would
    make the kernels read or write past its end)."""
    import torch
    x = torch.zeros((4, 64), dtype=torch.float32)
    cases = [
        (lambda: S.quantize_q8_1(x.half()), "float16"),
        (lambda: S.quantize_q8_1(x.t()), "contiguous"),
        (lambda: S.quantize_q8_1(x), "not a GPU"),
        (lambda: S.residual_rmsnorm(x.double()), "float64"),
        (lambda: S.combine(x[:, ::2], None), "contiguous"),
        (lambda: S.dispatch(torch.zeros((4, 2), dtype=torch.int64), 8), "int64"),
        (lambda: S.router_topk(torch.zeros(8), 2), "(tokens, experts)"),
        (lambda: S.mmvq(S.Q2_0, torch.zeros(10, dtype=torch.uint8), None, 128, 4), "elements"),
    ]
    for fn, why in cases:
        with pytest.raises(S.SmoeError) as e:
            fn()
        assert why in str(e.value), (why, str(e.value))


def test_native_shared_geometry_refusals():
    """A shared expert in its own native types: rows must be whole blocks of each projection's type, n_ff_shared a
    multiple of 32, every type one with a GEMV here; the workspace query refuses (returns 0) otherwise."""
    L = S.lib()
    ok = S.Geom(sh_type=S.Q3_K, sh_down_type=S.IQ4_NL)
    assert L.smoe_workspace_bytes(C.byref(ok.c()), 4) > 0
    for kw in (dict(sh_type=S.Q4_K, n_ff_shared=640),       # Q4_K down rows of 640 values: not whole 256-blocks
               dict(sh_type=S.Q8_0, n_ff_shared=48),        # n_ff_shared not a multiple of 32
               dict(sh_type=S.Q8_0, sh_down_type=1),        # F16: no GEMV here
               dict(sh_type=S.Q2_0, sh_gate_type=S.IQ2_S, n_embd=4096)):  # IQ2_S rows of 4096
        g = S.Geom(**kw)
        assert L.smoe_workspace_bytes(C.byref(g.c()), 4) == 0, kw
