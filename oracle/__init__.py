"""oracle - CPU restatement of StrataMetal's quantized MoE block (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only
as the checker or the timed CPU baseline.  The product path (stratametal_amd) never imports it.

The C library (oracle/liboracle.so, built by oracle/Makefile) holds the arithmetic; this module wraps it
for numpy arrays.  `ref()` loads oracle/_ref/libsmoe_ref.so, the reference's own header-only codecs
compiled from /root/reference (None when that build is absent).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

Q2_0 = 42
IQ2_S = 22


def build(quiet: bool = True) -> None:
    """Compile oracle/liboracle.so, its sanitized twin oracle/_asan/liboracle.so, and oracle/_ref where the reference
    tree exists."""
    out = subprocess.run(["make", "-C", _HERE, "all"], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if not quiet:
        print(out.stdout)


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def lib():
    global _LIB
    if _LIB is None:
        # SMOE_ORACLE_LIB: another build of the same library (the sanitized oracle/_asan/liboracle.so)
        path = os.environ.get("SMOE_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        _set_sigs(L)
        _LIB = L
    return _LIB


def _set_sigs(L):
    vp, i64, i32, u64, f32 = C.c_void_p, C.c_int64, C.c_int, C.c_uint64, C.c_float
    sigs = {
        "or_f16_from_f32": (C.c_uint16, [f32]),
        "or_f32_from_f16": (f32, [C.c_uint16]),
        "or_bf16_from_f32": (C.c_uint16, [f32]),
        "or_f32_from_bf16": (f32, [C.c_uint16]),
        "or_f16_from_f32_n": (None, [vp, i64, vp]),
        "or_f32_from_f16_n": (None, [vp, i64, vp]),
        "or_bf16_from_f32_n": (None, [vp, i64, vp]),
        "or_expf": (f32, [f32]),
        "or_logf": (f32, [f32]),
        "or_cos2pi": (f32, [f32]),
        "or_hash": (u64, [u64, u64, u64]),
        "or_uniform": (f32, [u64, u64, u64]),
        "or_normal": (f32, [u64, u64, u64]),
        "or_gen_normal": (None, [u64, u64, i64, f32, vp]),
        "or_gen_bf16": (None, [u64, u64, i64, f32, vp]),
        "or_gen_q2_0": (None, [u64, u64, i64, f32, vp]),
        "or_gen_iq2_s": (None, [u64, u64, i64, f32, vp]),
        "or_dequant_q2_0": (None, [vp, i64, vp]),
        "or_quant_q8_1": (None, [vp, i64, vp]),
        "or_q2_0_gemv_dev": (None, [vp, vp, i32, i32, vp]),
        "or_q2_0_gemv_ref": (None, [vp, vp, i32, i32, vp]),
        "or_q2_0_gemv_exact": (None, [vp, vp, i32, i32, vp]),
        "or_q2_0_gemv_no_minus_one": (None, [vp, vp, i32, i32, vp]),
        "or_iq2s_grid": (None, [vp]),
        "or_iq2_s_gemv_dev": (None, [vp, vp, i32, i32, vp]),
        "or_iq2_s_gemv_ref": (None, [vp, vp, i32, i32, vp]),
        "or_bf16_gemv_dev": (None, [vp, vp, i32, i32, vp]),
        "or_bf16_gemv_double": (None, [vp, vp, i32, i32, vp]),
        "or_f32_gemv_dev": (None, [vp, vp, i32, i32, vp]),
        "or_router_margin_dev": (i32, [vp, i32, i32, i32, vp, vp]),
        "or_f32_gemv_double": (None, [vp, vp, i32, i32, vp]),
        "or_route_dev": (None, [vp, i32, i32, i32, vp, vp]),
        "or_route_ref": (None, [vp, i32, i32, i32, vp, vp]),
        "or_swiglu_q8": (None, [vp, vp, i64, vp]),
        "or_silu_mul": (f32, [f32, f32]),
        "or_sigmoid": (f32, [f32]),
        "or_combine_dev": (None, [vp, vp, vp, i32, i32, vp]),
        "or_residual_rmsnorm_dev": (None, [vp, vp, i32, i32, C.c_float, vp]),
        "or_combine_double": (None, [vp, vp, vp, i32, i32, vp]),
        "or_dispatch": (None, [vp, i32, i32, i32, vp, vp, vp, vp]),
        "or_moe_decode_dev": (i32, [vp, vp, vp, i32, vp, i32, vp, i32]),
        "or_moe_decode_ref": (i32, [vp, vp, vp, i32, vp, i32, i32]),
        "or_moe_prefill": (i32, [vp, vp, vp, i32, vp, i32, vp, i32]),
        "or_moe_prefill_logits": (i32, [vp, vp, vp, i32, vp, vp, vp, i32, vp, i32]),
        "or_moe_decode_pool": (i32, [vp, vp, vp, i32, vp, i32, i32]),
        "or_hc_read_dev": (i32, [vp, i32, i32, i32, i32, f32, vp, vp, vp, vp, vp, vp]),
        "or_hc_read_ref": (i32, [vp, i32, i32, i32, i32, f32, vp, vp, vp, vp, i32, vp, vp]),
        "or_hc_write_dev": (None, [vp, vp, vp, i32, i32, i32, vp]),
        "or_row_bytes": (i64, [i32, i64]),
        "or_native_type": (i32, [i32]),
        "or_native_row_bytes": (i64, [i32, i64]),
        "or_native_dequant": (i32, [i32, vp, i64, vp]),
        "or_native_part": (f32, [i32, vp, vp, i32]),
        "or_native_gemv": (i32, [i32, vp, vp, i32, i32, i32, vp]),
        "or_native_gemv_double": (i32, [i32, vp, vp, i32, i32, i32, vp]),
        "or_expert_group": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp]),
        "or_expert_dev": (i32, [i32, vp, i32, i32, vp, vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def ref():
    """The reference's own header-only codecs (oracle/_ref), or None if that build is absent."""
    global _REF
    if _REF is None:
        path = os.path.join(_HERE, "_ref", "libsmoe_ref.so")
        if not os.path.exists(path):
            return None
        R = C.CDLL(path)
        R.ref_f16_from_f32.restype = C.c_uint16
        R.ref_f16_from_f32.argtypes = [C.c_float]
        R.ref_f32_from_f16.restype = C.c_float
        R.ref_f32_from_f16.argtypes = [C.c_uint16]
        R.ref_bf16_from_f32.restype = C.c_uint16
        R.ref_bf16_from_f32.argtypes = [C.c_float]
        for n in ("ref_f16_from_f32_n", "ref_bf16_from_f32_n", "ref_dequantize_q2_0"):
            getattr(R, n).restype = None
            getattr(R, n).argtypes = [C.c_void_p, C.c_int64, C.c_void_p]
        R.ref_f32_from_f16_all.restype = None
        R.ref_f32_from_f16_all.argtypes = [C.c_void_p]
        R.ref_iq2s_grid.restype = None
        R.ref_iq2s_grid.argtypes = [C.c_void_p]
        R.ref_dequantize.restype = C.c_int
        R.ref_dequantize.argtypes = [C.c_int, C.c_void_p, C.c_int64, C.c_void_p]
        R.ref_gguf_list.restype = C.c_int
        R.ref_gguf_list.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
        _REF = R
    return _REF


# ------------------------------------------------------------------------------------------------ codecs

def f16_from_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().or_f16_from_f32_n(_p(x), x.size, _p(y))
    return y


def f32_from_f16(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().or_f32_from_f16_n(_p(h), h.size, _p(y))
    return y


def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().or_bf16_from_f32_n(_p(x), x.size, _p(y))
    return y


def f32_from_bf16(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def row_bytes(wtype: int, n: int) -> int:
    return int(lib().or_row_bytes(wtype, n))


# ------------------------------------------------------------------------------------------------ generators

def gen_normal(seed: int, stream: int, n: int, sigma: float = 1.0) -> np.ndarray:
    y = np.empty(n, np.float32)
    lib().or_gen_normal(seed, stream, n, sigma, _p(y))
    return y


def gen_bf16(seed: int, stream: int, n: int, sigma: float) -> np.ndarray:
    y = np.empty(n, np.uint16)
    lib().or_gen_bf16(seed, stream, n, sigma, _p(y))
    return y


def gen_q2_0(seed: int, stream: int, n_blocks: int, sigma: float = 0.02) -> np.ndarray:
    y = np.empty(n_blocks * 18, np.uint8)
    lib().or_gen_q2_0(seed, stream, n_blocks, sigma, _p(y))
    return y


def gen_iq2_s(seed: int, stream: int, n_blocks: int, sigma: float = 0.02) -> np.ndarray:
    y = np.empty(n_blocks * 82, np.uint8)
    lib().or_gen_iq2_s(seed, stream, n_blocks, sigma, _p(y))
    return y


# The other native GGUF types: (values per block, bytes per block, fp16 scale fields, scale divisor) -- the divisor
# keeps the dequantised weights near sigma (a block value is d times a code of this size).
Q8_0, Q4_0, Q5_0, IQ4_NL, IQ4_XS, Q3_K, Q4_K, Q5_K, Q6_K = 8, 2, 6, 20, 23, 11, 12, 13, 14
NATIVE = {Q8_0: (32, 34, (0,), 64.0), Q4_0: (32, 18, (0,), 8.0), Q5_0: (32, 22, (0,), 16.0),
          IQ4_NL: (32, 18, (0,), 64.0), IQ4_XS: (256, 136, (0,), 2000.0), Q3_K: (256, 110, (108,), 100.0),
          Q4_K: (256, 144, (0, 2), 500.0), Q5_K: (256, 176, (0, 2), 500.0), Q6_K: (256, 210, (208,), 2000.0)}


def gen_native_blocks(wtype: int, seed: int, stream: int, n_values: int, sigma: float = 0.02) -> np.ndarray:
    """Random blocks of a native type: uniform code and scale bytes, fp16 scale fields RNE-fp16 of
    |N(0, sigma / divisor)| (no inf or NaN scales).  numpy's PCG64 seeded from (seed, stream)."""
    qk, nb, fields, div = NATIVE[wtype]
    assert n_values % qk == 0
    n_blocks = n_values // qk
    rng = np.random.Generator(np.random.PCG64([seed, stream, wtype]))
    b = rng.integers(0, 256, size=(n_blocks, nb), dtype=np.uint8)
    for f in fields:
        d = f16_from_f32(np.abs(rng.normal(0.0, sigma / div, n_blocks)).astype(np.float32))
        b[:, f:f + 2] = d.view(np.uint8).reshape(n_blocks, 2)
    return b.ravel()


def gen_blocks(wtype: int, seed: int, stream: int, n_values: int, sigma: float = 0.02) -> np.ndarray:
    if wtype == Q2_0:
        return gen_q2_0(seed, stream, n_values // 64, sigma)
    if wtype == IQ2_S:
        return gen_iq2_s(seed, stream, n_values // 256, sigma)
    if wtype in NATIVE:
        return gen_native_blocks(wtype, seed, stream, n_values, sigma)
    raise ValueError(wtype)


def native_row_bytes(wtype: int, n: int) -> int:
    return int(lib().or_native_row_bytes(wtype, n))


def native_dequant(wtype: int, blocks: np.ndarray, n_values: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty(n_values, np.float32)
    assert lib().or_native_dequant(wtype, _p(blocks), n_values, _p(y)) == 0
    return y


def ref_dequantize(wtype: int, blocks: np.ndarray, n_values: int) -> Optional[np.ndarray]:
    """The reference's own dequantiser (oracle/_ref), or None when that build is absent."""
    R = ref()
    if R is None:
        return None
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    y = np.empty(n_values, np.float32)
    assert R.ref_dequantize(wtype, _p(blocks), n_values, _p(y)) == 0
    return y


def native_gemv(wtype: int, w, xq, n_in: int, n_out: int, n_col: int = 1, double: bool = False) -> np.ndarray:
    """y[c][r] for n_col q8_1 columns: the 32-lane MMVQ order (or, with double, the dequantised double sums)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    y = np.empty((n_col, n_out), np.float32)
    fn = lib().or_native_gemv_double if double else lib().or_native_gemv
    assert fn(wtype, _p(w), _p(xq), n_in, n_out, n_col, _p(y)) == 0
    return y


# ------------------------------------------------------------------------------------------------ kernels

def dequant_q2_0(blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    nb = blocks.size // 18
    y = np.empty(nb * 64, np.float32)
    lib().or_dequant_q2_0(_p(blocks), nb, _p(y))
    return y


def quant_q8_1(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    y = np.empty(x.size // 32 * 36, np.uint8)
    lib().or_quant_q8_1(_p(x), x.size, _p(y))
    return y


def _gemv(fn, w, xq, n_in, n_out, dtype=np.float32):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    y = np.empty(n_out, dtype)
    fn(_p(w), _p(xq), n_in, n_out, _p(y))
    return y


def q2_0_gemv_dev(w, xq, n_in, n_out):
    return _gemv(lib().or_q2_0_gemv_dev, w, xq, n_in, n_out)


def q2_0_gemv_ref(w, xq, n_in, n_out):
    return _gemv(lib().or_q2_0_gemv_ref, w, xq, n_in, n_out)


def q2_0_gemv_exact(w, xq, n_in, n_out):
    return _gemv(lib().or_q2_0_gemv_exact, w, xq, n_in, n_out, np.float64)


def q2_0_gemv_no_minus_one(w, xq, n_in, n_out):
    return _gemv(lib().or_q2_0_gemv_no_minus_one, w, xq, n_in, n_out)


def iq2_s_gemv_dev(w, xq, n_in, n_out):
    return _gemv(lib().or_iq2_s_gemv_dev, w, xq, n_in, n_out)


def iq2_s_gemv_ref(w, xq, n_in, n_out):
    return _gemv(lib().or_iq2_s_gemv_ref, w, xq, n_in, n_out)


def gemv_dev(wtype, w, xq, n_in, n_out):
    return (iq2_s_gemv_dev if wtype == IQ2_S else q2_0_gemv_dev)(w, xq, n_in, n_out)


def iq2s_grid() -> np.ndarray:
    g = np.empty(1024, np.uint64)
    lib().or_iq2s_grid(_p(g))
    return g


def bf16_gemv_dev(xb, w, n_in, n_out):
    xb = np.ascontiguousarray(xb, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    y = np.empty(n_out, np.float32)
    lib().or_bf16_gemv_dev(_p(xb), _p(w), n_in, n_out, _p(y))
    return y


def bf16_gemv_double(xb, w, n_in, n_out):
    xb = np.ascontiguousarray(xb, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    y = np.empty(n_out, np.float32)
    lib().or_bf16_gemv_double(_p(xb), _p(w), n_in, n_out, _p(y))
    return y


def f32_gemv_dev(x, w, n_in, n_out):
    """The f32 router's device order (router_dtype 1): 4-element chunks per lane, fused multiply-adds."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty(n_out, np.float32)
    lib().or_f32_gemv_dev(_p(x), _p(w), n_in, n_out, _p(y))
    return y


def f32_gemv_double(x, w, n_in, n_out):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty(n_out, np.float32)
    lib().or_f32_gemv_double(_p(x), _p(w), n_in, n_out, _p(y))
    return y


def _route(fn, logits, k):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    if logits.ndim == 1:
        logits = logits[None, :]
    T, E = logits.shape
    ids = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    fn(_p(logits), T, E, k, _p(ids), _p(w))
    return ids, w


def router_margin_dev(logits, k):
    """The router-margin diagnostic in the device order: stats [T][4] = (p_k - p_k1, logit gap, p_k, p_k1) and
    ids [T][2] = (id_k, id_k1) of the k-th and (k+1)-th experts by probability."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    stats = np.empty((T, 4), np.float32)
    ids = np.empty((T, 2), np.int32)
    if lib().or_router_margin_dev(_p(logits), T, E, k, _p(stats), _p(ids)) != 0:
        raise ValueError("router margin needs 1 <= k < n_expert")
    return stats, ids


def route_dev(logits, k):
    return _route(lib().or_route_dev, logits, k)


def route_ref(logits, k):
    return _route(lib().or_route_ref, logits, k)


def swiglu_q8(gate, up):
    gate = np.ascontiguousarray(gate, dtype=np.float32).ravel()
    up = np.ascontiguousarray(up, dtype=np.float32).ravel()
    y = np.empty(gate.size // 32 * 36, np.uint8)
    lib().or_swiglu_q8(_p(gate), _p(up), gate.size, _p(y))
    return y


def combine_dev(parts, w, shared):
    parts = np.ascontiguousarray(parts, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    k, n = parts.shape
    y = np.empty(n, np.float32)
    sh = None if shared is None else np.ascontiguousarray(shared, dtype=np.float32)
    lib().or_combine_dev(_p(parts), _p(w), None if sh is None else _p(sh), n, k, _p(y))
    return y


def residual_rmsnorm_dev(x, r=None, eps: float = 1e-6):
    """RMSNorm(x + r) per row, unit weight, in the device's order (the stacked configuration's junction)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    rr = None if r is None else np.ascontiguousarray(r, dtype=np.float32)
    out = np.empty_like(x)
    lib().or_residual_rmsnorm_dev(_p(x), None if rr is None else _p(rr), x.size // n, n, eps, _p(out))
    return out


def combine_double(parts, w, shared):
    parts = np.ascontiguousarray(parts, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    k, n = parts.shape
    y = np.empty(n, np.float32)
    sh = None if shared is None else np.ascontiguousarray(shared, dtype=np.float32)
    lib().or_combine_double(_p(parts), _p(w), None if sh is None else _p(sh), n, k, _p(y))
    return y


def dispatch(ids, n_expert):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, k = ids.shape
    counts = np.empty(n_expert, np.int32)
    offsets = np.empty(n_expert + 1, np.int32)
    perm = np.empty(T * k, np.int32)
    slot = np.empty(T * k, np.int32)
    lib().or_dispatch(_p(ids), T, k, n_expert, _p(counts), _p(offsets), _p(perm), _p(slot))
    return counts, offsets, perm, slot


# ------------------------------------------------------------------------------------------------ the block

class _Geom(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_embd", "n_ff", "n_ff_shared", "n_expert", "top_k", "w_type", "sh_type",
                                         "router_dtype", "sh_gate_type", "sh_up_type", "sh_down_type")]


class _Weights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("gate_exps", "up_exps", "down_exps", "router", "gate_sh", "up_sh",
                                          "down_sh", "gate_inp_sh", "logit_bias")]


class _Trace(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("logits", "ids", "weights", "counts", "offsets", "perm", "slot", "xq",
                                          "hq", "parts", "shared", "sgate")]


@dataclass
class Geom:
    n_embd: int = 2048
    n_ff: int = 512
    n_ff_shared: int = 512
    n_expert: int = 512
    top_k: int = 10
    w_type: int = Q2_0
    sh_type: int = Q2_0
    router_dtype: int = 0
    sh_gate_type: int = 0  # the shared expert's projections in their own native types (0: sh_type)
    sh_up_type: int = 0
    sh_down_type: int = 0

    def c(self):
        return _Geom(self.n_embd, self.n_ff, self.n_ff_shared, self.n_expert, self.top_k, self.w_type, self.sh_type,
                     self.router_dtype, self.sh_gate_type, self.sh_up_type, self.sh_down_type)

    def shared_types(self):
        """(gate, up, down) types of the shared expert."""
        return tuple(t if t else self.sh_type for t in (self.sh_gate_type, self.sh_up_type, self.sh_down_type))


@dataclass
class Weights:
    gate_exps: np.ndarray
    up_exps: np.ndarray
    down_exps: np.ndarray
    router: np.ndarray           # uint16 bf16 [E][H], or f32 [E][H] when router_dtype is 1
    gate_sh: Optional[np.ndarray] = None
    up_sh: Optional[np.ndarray] = None
    down_sh: Optional[np.ndarray] = None
    gate_inp_sh: Optional[np.ndarray] = None  # uint16 bf16 [H]
    logit_bias: Optional[np.ndarray] = None   # f32 [E]

    def c(self):
        def ptr(a):
            return None if a is None else a.ctypes.data
        return _Weights(ptr(self.gate_exps), ptr(self.up_exps), ptr(self.down_exps), ptr(self.router),
                        ptr(self.gate_sh), ptr(self.up_sh), ptr(self.down_sh), ptr(self.gate_inp_sh),
                        ptr(self.logit_bias))


def make_weights(g: Geom, seed: int, n_expert_alloc: Optional[int] = None, zipf_bias: Optional[np.ndarray] = None,
                 sigma: float = 0.02) -> Weights:
    """Synthetic layer weights from the counter RNG.  Stream ids: 1 gate, 2 up, 3 down, 4 router, 5/6/7 shared
    gate/up/down, 8 shared gate_inp.  The device generator (smoe_synth_*) uses the same streams."""
    E = g.n_expert if n_expert_alloc is None else n_expert_alloc
    H, F, Fs = g.n_embd, g.n_ff, g.n_ff_shared
    gate = gen_blocks(g.w_type, seed, 1, E * F * H, sigma)
    up = gen_blocks(g.w_type, seed, 2, E * F * H, sigma)
    down = gen_blocks(g.w_type, seed, 3, E * H * F, sigma)
    # the router is generated in f32 and stored as bf16 (the repo's contract) unless router_dtype is 1
    router = gen_normal(seed, 4, E * H, sigma) if g.router_dtype == 1 else gen_bf16(seed, 4, E * H, sigma)
    w = Weights(gate, up, down, router)
    if g.sh_type >= 0:
        tg, tu, td = g.shared_types()
        w.gate_sh = gen_blocks(tg, seed, 5, Fs * H, sigma)
        w.up_sh = gen_blocks(tu, seed, 6, Fs * H, sigma)
        w.down_sh = gen_blocks(td, seed, 7, H * Fs, sigma)
        w.gate_inp_sh = gen_bf16(seed, 8, H, sigma)
    if zipf_bias is not None:
        w.logit_bias = np.ascontiguousarray(zipf_bias, dtype=np.float32)
    return w


def _run_block(fn, g: Geom, w: Weights, x: np.ndarray, add_shared: bool, trace: bool, n_threads: int, with_trace=True):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    y = np.empty_like(x)
    gc, wc = g.c(), w.c()
    tr = None
    out = {}
    if trace and with_trace:
        H, E, K, F = g.n_embd, g.n_expert, g.top_k, g.n_ff
        out = dict(logits=np.empty((T, E), np.float32), ids=np.empty((T, K), np.int32),
                   weights=np.empty((T, K), np.float32), counts=np.empty(E, np.int32),
                   offsets=np.empty(E + 1, np.int32), perm=np.empty(T * K, np.int32), slot=np.empty(T * K, np.int32),
                   xq=np.empty(T * H // 32 * 36, np.uint8), hq=np.empty(T * K * F // 32 * 36, np.uint8),
                   parts=np.empty((T * K, H), np.float32), shared=np.empty((T, H), np.float32),
                   sgate=np.empty(T, np.float32))
        tr = _Trace(*[out[n].ctypes.data for n in ("logits", "ids", "weights", "counts", "offsets", "perm", "slot",
                                                   "xq", "hq", "parts", "shared", "sgate")])
    if with_trace:
        rc = fn(C.byref(gc), C.byref(wc), _p(x), T, _p(y), int(add_shared), None if tr is None else C.byref(tr),
                n_threads)
    else:
        rc = fn(C.byref(gc), C.byref(wc), _p(x), T, _p(y), int(add_shared), n_threads)
    if rc != 0:
        raise ValueError(f"oracle rejected the block (rc={rc})")
    return (y, out) if trace else y


def moe_decode_dev(g, w, x, add_shared=True, trace=False, n_threads=1):
    return _run_block(lib().or_moe_decode_dev, g, w, x, add_shared, trace, n_threads)


def moe_decode_ref(g, w, x, add_shared=True, n_threads=1):
    return _run_block(lib().or_moe_decode_ref, g, w, x, add_shared, False, n_threads, with_trace=False)


def moe_decode_pool(g, w, x, add_shared=True, n_threads=1, library=None):
    """The decode contract as the pooled CPU baseline computes it (bitwise equal to moe_decode_dev).  `library`:
    another build of the oracle (bench.py's -march=native one) with the same signatures."""
    L = lib() if library is None else library
    return _run_block(L.or_moe_decode_pool, g, w, x, add_shared, False, n_threads, with_trace=False)


def load_library(path: str):
    """A build of the oracle at `path` (e.g. `make native OUT=path`), with the signatures set as in lib()."""
    L = C.CDLL(path)
    _set_sigs(L)
    return L


def moe_prefill(g, w, x, add_shared=True, trace=False, n_threads=1, logits=None, sgate=None):
    """The prefill contract.  With `logits` ([T][E], bias included) and `sgate` ([T]) the router's outputs are taken
    as given -- the device's own, whose matrix-core sums are in the hardware's order -- and routed in the device
    order."""
    if logits is None:
        return _run_block(lib().or_moe_prefill, g, w, x, add_shared, trace, n_threads)
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    sgv = None if sgate is None else np.ascontiguousarray(sgate, dtype=np.float32)
    assert lg.shape == (np.asarray(x).shape[0], g.n_expert)

    def fn(gc, wc, xp, T, yp, add, trp, nth):
        return lib().or_moe_prefill_logits(gc, wc, xp, T, _p(lg), None if sgv is None else _p(sgv), yp, add, trp, nth)
    return _run_block(fn, g, w, x, add_shared, trace, n_threads)


# ------------------------------------------------------------------------------------------------ metrics

def rel_l1_rows(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    """Per-row sum|a-b| / sum|b| (metal/src/pack_parity.cpp:2425-2433, metal/src/iq_parity.cpp:306-313)."""
    got = np.atleast_2d(np.asarray(got, np.float64))
    want = np.atleast_2d(np.asarray(want, np.float64))
    num = np.abs(got - want).sum(axis=1)
    den = np.abs(want).sum(axis=1)
    return np.where(den > 0, num / np.where(den > 0, den, 1.0), np.where(num == 0, 0.0, 1.0))


# ------------------------------------------------------------------------------------------------ layer ends

@dataclass
class HcWeights:
    """The hyper-connection tensors of one layer: norm [hc][n] f32 (the stored 1 + w), down [hc_lr][hc n], up
    [hc n][hc_lr] and inject [hc][hc n] bf16 bits."""
    hc: int
    hc_lr: int
    eps: float
    norm: np.ndarray
    down: np.ndarray
    up: np.ndarray
    inject: np.ndarray


def make_hc(n: int, hc: int, hc_lr: int, seed: int, eps: float = 1e-6) -> HcWeights:
    """Seeded hyper-connection tensors: norm = 1 + 0.1 N(0,1) in f32, down/up N(0, 0.2^2), inject N(0, 0.05^2) as bf16
    (the reference test's fixture scales, metal/src/gr_parity.cpp:170-200), from the counter generator."""
    hd = hc * n
    norm = (np.float32(1.0) + gen_normal(seed, 30, hd, 0.1)).astype(np.float32)
    return HcWeights(hc, hc_lr, eps, norm, gen_bf16(seed, 31, hc_lr * hd, 0.2), gen_bf16(seed, 32, hd * hc_lr, 0.2),
                     gen_bf16(seed, 33, hc * hd, 0.05))


def hc_read_dev(R: np.ndarray, n: int, w: HcWeights):
    R = np.ascontiguousarray(R, dtype=np.float32)
    T = R.size // (w.hc * n)
    mixed = np.empty((T, n), np.float32)
    inject = np.empty((T, w.hc), np.float32)
    rc = lib().or_hc_read_dev(_p(R), T, n, w.hc, w.hc_lr, w.eps, _p(w.norm), _p(w.down), _p(w.up), _p(w.inject),
                              _p(mixed), _p(inject))
    if rc != 0:
        raise ValueError("oracle rejected the hyper-connection shape")
    return mixed, inject


def hc_read_ref(R: np.ndarray, n: int, w: HcWeights, round_act: bool = True):
    R = np.ascontiguousarray(R, dtype=np.float32)
    T = R.size // (w.hc * n)
    mixed = np.empty((T, n), np.float32)
    inject = np.empty((T, w.hc), np.float32)
    rc = lib().or_hc_read_ref(_p(R), T, n, w.hc, w.hc_lr, w.eps, _p(w.norm), _p(w.down), _p(w.up), _p(w.inject),
                              int(round_act), _p(mixed), _p(inject))
    if rc != 0:
        raise ValueError("oracle rejected the hyper-connection shape")
    return mixed, inject


def hc_write_dev(R: np.ndarray, y: np.ndarray, inject: np.ndarray, n: int, hc: int):
    R = np.ascontiguousarray(R, dtype=np.float32)
    y = np.ascontiguousarray(y, dtype=np.float32)
    inject = np.ascontiguousarray(inject, dtype=np.float32)
    T = R.size // (hc * n)
    out = np.empty_like(R)
    lib().or_hc_write_dev(_p(R), _p(y), _p(inject), T, n, hc, _p(out))
    return out


def ref_gguf_list(path: str):
    """The reference reader's listing of a GGUF model (oracle/_ref): (status, text), or None without _ref."""
    R = ref()
    if R is None:
        return None
    buf = C.create_string_buffer(1 << 20)
    rc = R.ref_gguf_list(path.encode(), buf, 1 << 20)
    return rc, buf.value.decode()


# ---- the expert tier (smoe_cache.c)

def expert_group(ids: np.ndarray, kpt: int, n_expert: int, resident: np.ndarray) -> Dict:
    """The oracle's hit/miss split and grouping: grp_expert, grp_start, ent_dst, ent_tok, miss_dst, counts."""
    ids = np.ascontiguousarray(ids, dtype=np.int32).ravel()
    res = np.ascontiguousarray(resident, dtype=np.uint8)
    n = ids.size
    G = max(1, min(n, n_expert))
    out = dict(grp_expert=np.full(G, -1, np.int32), grp_start=np.zeros(G + 1, np.int32),
               ent_dst=np.full(max(n, 1), -1, np.int32), ent_tok=np.full(max(n, 1), -1, np.int32),
               miss_dst=np.full(max(n, 1), -1, np.int32), counts=np.zeros(4, np.int32))
    rc = lib().or_expert_group(_p(ids), n, kpt, n_expert, _p(res), _p(out["grp_expert"]), _p(out["grp_start"]),
                               _p(out["ent_dst"]), _p(out["ent_tok"]), _p(out["miss_dst"]), _p(out["counts"]))
    if rc != 0:
        raise ValueError("or_expert_group refused its arguments")
    return out


def expert_blob(g, w, e: int) -> np.ndarray:
    """Expert e's blob [gate rows | up rows | down rows] from the planes of the host weights."""
    gu = row_bytes(g.w_type, g.n_embd) * g.n_ff
    dn = row_bytes(g.w_type, g.n_ff) * g.n_embd
    return np.concatenate([w.gate_exps[e * gu:(e + 1) * gu], w.up_exps[e * gu:(e + 1) * gu],
                           w.down_exps[e * dn:(e + 1) * dn]])


def expert_dev(wtype: int, blob: np.ndarray, H: int, F: int, xq_row: np.ndarray) -> np.ndarray:
    """One routed expert on one token's q8_1 row under the decode contract."""
    out = np.empty(H, np.float32)
    b = np.ascontiguousarray(blob, dtype=np.uint8)
    x = np.ascontiguousarray(xq_row, dtype=np.uint8)
    if lib().or_expert_dev(wtype, _p(b), H, F, _p(x), _p(out)) != 0:
        raise ValueError("or_expert_dev: type is not Q2_0 or IQ2_S")
    return out

