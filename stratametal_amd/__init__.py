"""stratametal_amd - MI355X (gfx950) quantized mixture-of-experts block.

Python host binding of the C ABI in include/smoe.h (libsmoe.so, built by stratametal_amd/build.py).  The
arithmetic lives in the HIP kernels; this module only passes device pointers (torch tensors supply the
memory and the stream) and turns refused calls into exceptions, as the reference's wrappers throw
MetalError (metal/include/strata/metal/device.hpp:28-31).  There is no CPU fallback: without the built
library every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import functools
import os
from dataclasses import dataclass
from typing import Dict, Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
# SMOE_LIB names another build of the same library (the host-sanitized lib/libsmoe_asan.so, for tests/test_sanitize.py)
LIB_PATH = os.environ.get("SMOE_LIB") or os.path.join(_HERE, "lib", "libsmoe.so")
_LIB = None

Q2_0 = 42
IQ2_S = 22
PATH_AUTO, PATH_GEMV, PATH_MFMA = 0, 1, 2
ROUTER_BF16, ROUTER_F32 = 0, 1  # smoe_geom.router_dtype
MFMA_TOKENS = 128  # SMOE_PATH_AUTO runs the prefill (MFMA) contract from this many tokens on
MFMA_CHUNK = 128   # columns per MFMA work item

_STATUS = {0: "ok", -1: "invalid argument", -2: "buffer too small", -3: "unsupported ggml type",
           -4: "HIP runtime error", -5: "misaligned pointer", -6: "NULL pointer"}


class SmoeError(RuntimeError):
    """A call the library refused (status != SMOE_OK); `.status` is the smoe_status code."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"{_STATUS.get(status, status)}: {msg}")
        self.status = status


class _Geom(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_embd", "n_ff", "n_ff_shared", "n_expert", "top_k", "w_type", "sh_type",
                                         "router_dtype", "sh_gate_type", "sh_up_type", "sh_down_type")]


class _Weights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("gate_exps", "up_exps", "down_exps", "router", "gate_sh", "up_sh",
                                          "down_sh", "gate_inp_sh", "logit_bias")]


class _Trace(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("logits", "ids", "weights", "counts", "offsets", "perm", "slot", "sgate",
                                          "stage_events", "xq", "hq", "parts", "shared", "overflow", "egate", "eup",
                                          "sgu", "shq")]

class _Hc(C.Structure):
    _fields_ = [("hc", C.c_int32), ("hc_lr", C.c_int32), ("eps", C.c_float), ("norm", C.c_void_p),
                ("down", C.c_void_p), ("up", C.c_void_p), ("inject", C.c_void_p)]


STAGES = ("router", "route", "gate_up", "down", "combine")
STATUS_X_FP16, STATUS_H_FP16, STATUS_WAIT = 1, 2, 4  # bits of a call's status mask (smoe.h SMOE_STATUS_*)


def set_wait_limit(polls: int) -> int:
    """The bound of the fused decode launch's waits (smoe_set_wait_limit): polls > 0 sets it, 0 restores the default,
    a negative value makes every wait give up at once (tests of the give-up path).  Returns the previous bound."""
    return int(lib().smoe_set_wait_limit(int(polls)))
STAGE_EVENTS = len(STAGES) + 1


def lib():
    """The loaded libsmoe.so.  Raises ImportError when it has not been built (no fallback exists)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m stratametal_amd.build`")
        L = C.CDLL(LIB_PATH)
        vp, i32, i64, u64, f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_float
        sigs = {
            "smoe_workspace_bytes": (C.c_size_t, [vp, i32]),
            "smoe_forward": (i32, [vp, vp, vp, i32, vp, i32, vp, C.c_size_t, vp, vp]),
            "smoe_forward_path": (i32, [vp, vp, vp, i32, vp, i32, vp, C.c_size_t, vp, i32, vp]),
            "smoe_forward_residual": (i32, [vp, vp, vp, vp, f32, vp, i32, vp, i32, vp, C.c_size_t, vp, vp]),
            "smoe_forward_static": (i32, [vp, vp, vp, i32, vp, i32, vp, vp]),
            "smoe_forward_status": (i32, [vp, vp, vp]),
            "smoe_set_wait_limit": (i32, [i32]),
            "smoe_hc_read_workspace_bytes": (C.c_size_t, [vp, i32, i32]),
            "smoe_hc_read": (i32, [vp, i32, vp, i32, vp, vp, vp, C.c_size_t, vp]),
            "smoe_hc_write": (i32, [vp, i32, vp, vp, vp, i32, vp, vp]),
            "smoe_ffn_workspace_bytes": (C.c_size_t, [vp, vp, i32]),
            "smoe_ffn_run": (i32, [vp, vp, vp, vp, i32, vp, i32, vp, C.c_size_t, vp, vp]),
            "smoe_router_topk": (i32, [vp, i32, i32, i32, vp, vp, vp]),
            "smoe_router_margin": (i32, [vp, i32, i32, i32, vp, vp, vp]),
            "smoe_f32_to_bf16": (i32, [vp, i64, vp, vp]),
            "smoe_bf16_gemv": (i32, [vp, vp, vp, i32, i32, i32, vp]),
            "smoe_quantize_q8_1": (i32, [vp, i64, vp, vp]),
            "smoe_mmvq": (i32, [i32, vp, i64, vp, i32, i32, i32, vp, vp]),
            "smoe_swiglu_q8": (i32, [vp, vp, i64, vp, vp]),
            "smoe_combine": (i32, [vp, vp, vp, vp, i32, i32, vp]),
            "smoe_dispatch": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp]),
            "smoe_expert_bytes": (C.c_size_t, [i32, i32, i64, i64]),
            "smoe_residual_rmsnorm": (i32, [vp, vp, i32, i32, f32, vp, vp]),
            "smoe_expert_scratch_bytes": (C.c_size_t, [i64, i64, i64]),
            "smoe_expert": (i32, [vp, C.c_size_t, vp, i32, i32, i64, i64, i64, vp, vp, C.c_size_t, vp]),
            "smoe_synth_blocks": (i32, [i32, u64, u64, i64, f32, vp, vp]),
            "smoe_synth_bf16": (i32, [u64, u64, i64, f32, vp, vp]),
            "smoe_synth_normal": (i32, [u64, u64, i64, f32, vp, vp]),
            "smoe_status_str": (C.c_char_p, [i32]),
            "smoe_last_error": (C.c_char_p, []),
            "smoe_abi_version": (i32, []),
            "smoe_model_open": (i32, [C.c_char_p, C.POINTER(vp)]),
            "smoe_model_close": (None, [vp]),
            "smoe_model_n_shards": (i32, [vp]),
            "smoe_model_n_tensors": (i64, [vp]),
            "smoe_model_tensor": (i32, [vp, C.c_char_p, vp]),
            "smoe_model_tensor_at": (i32, [vp, i64, C.c_char_p, C.c_size_t, vp]),
            "smoe_model_meta_u64": (i32, [vp, C.c_char_p, C.POINTER(u64)]),
            "smoe_model_meta_str": (i32, [vp, C.c_char_p, C.c_char_p, C.c_size_t]),
            "smoe_layer_plan_for": (i32, [vp, i32, i32, i32, vp]),
            "smoe_layer_upload": (i32, [vp, vp, vp, C.c_size_t, vp, vp, vp]),
            "smoe_expert_blob_bytes": (C.c_size_t, [vp]),
            "smoe_expert_pack": (i32, [vp, vp, i32, vp, vp]),
            "smoe_expert_group": (i32, [vp, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp]),
            "smoe_expert_grouped_workspace_bytes": (C.c_size_t, [vp, i32, i32, i32]),
            "smoe_expert_grouped": (i32, [vp, vp, vp, vp, vp, vp, i32, i32, vp, i32, vp, i32, vp, C.c_size_t, vp]),
            "smoe_verify_workspace_bytes": (C.c_size_t, [vp, i32]),
            "smoe_verify_begin": (i32, [vp, vp, vp, vp, i32, vp, vp, vp, vp, vp, vp, C.c_size_t, vp]),
            "smoe_verify_end": (i32, [vp, i32, vp, vp, i32, vp, vp, C.c_size_t, vp]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _check(status: int):
    if status != 0:
        raise SmoeError(status, lib().smoe_last_error().decode())


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _need(t, name: str, dtype, shape=None, numel=None):
    """Refuse, before any launch, a tensor the kernels would misread or run past: it must be on a GPU, contiguous,
    of `dtype`, and (when given) of `shape` or at least `numel` elements."""
    import torch
    if not isinstance(t, torch.Tensor):
        raise SmoeError(-1, f"{name} is not a tensor")
    if t.dtype != dtype:
        raise SmoeError(-1, f"{name} is {t.dtype}, needs {dtype}")
    if not t.is_contiguous():
        raise SmoeError(-5, f"{name} is not contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise SmoeError(-2, f"{name} has shape {tuple(t.shape)}, needs {tuple(shape)}")
    if numel is not None and t.numel() < numel:
        raise SmoeError(-2, f"{name} has {t.numel()} elements, needs {numel}")
    if t.device.type != "cuda":
        raise SmoeError(-1, f"{name} is on {t.device}, not a GPU")
    return t


def _stream(stream=None) -> int:
    import torch
    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream


# the other native GGUF types (smoe.h): type -> (values per block, bytes per block)
Q8_0, Q4_0, Q5_0, IQ4_NL, IQ4_XS, Q3_K, Q4_K, Q5_K, Q6_K = 8, 2, 6, 20, 23, 11, 12, 13, 14
NATIVE_BLOCKS = {Q8_0: (32, 34), Q4_0: (32, 18), Q5_0: (32, 22), IQ4_NL: (32, 18), IQ4_XS: (256, 136),
                 Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}


def row_bytes(wtype: int, n: int) -> int:
    if wtype == Q2_0:
        return n // 64 * 18
    if wtype == IQ2_S:
        return n // 256 * 82
    if wtype in NATIVE_BLOCKS:
        qk, nb = NATIVE_BLOCKS[wtype]
        return n // qk * nb
    raise ValueError(wtype)


@dataclass
class Geom:
    """Layer geometry (smoe_geom).  Defaults are the benchmark configurations' layer."""
    n_embd: int = 2048
    n_ff: int = 512
    n_ff_shared: int = 512
    n_expert: int = 512
    top_k: int = 10
    w_type: int = Q2_0
    sh_type: int = Q2_0
    router_dtype: int = 0
    # the shared expert's gate, up and down projections in their own native types (0: sh_type)
    sh_gate_type: int = 0
    sh_up_type: int = 0
    sh_down_type: int = 0

    def c(self) -> _Geom:
        return _Geom(self.n_embd, self.n_ff, self.n_ff_shared, self.n_expert, self.top_k, self.w_type, self.sh_type,
                     self.router_dtype, self.sh_gate_type, self.sh_up_type, self.sh_down_type)

    def shared_types(self):
        """(gate, up, down) types of the shared expert."""
        return tuple(t if t else self.sh_type for t in (self.sh_gate_type, self.sh_up_type, self.sh_down_type))

    def expert_bytes(self) -> int:
        return 2 * self.n_ff * row_bytes(self.w_type, self.n_embd) + self.n_embd * row_bytes(self.w_type, self.n_ff)

    def shared_bytes(self) -> int:
        if self.sh_type < 0:
            return 0
        tg, tu, td = self.shared_types()
        return (self.n_ff_shared * (row_bytes(tg, self.n_embd) + row_bytes(tu, self.n_embd))
                + self.n_embd * row_bytes(td, self.n_ff_shared))


def workspace_bytes(g: Geom, max_tokens: int) -> int:
    n = lib().smoe_workspace_bytes(C.byref(g.c()), max_tokens)
    if n == 0:
        raise SmoeError(-1, lib().smoe_last_error().decode() or "bad geometry")
    return n


# ------------------------------------------------------------------------------------------------ layers

WEIGHT_NAMES = ("gate_exps", "up_exps", "down_exps", "router", "gate_sh", "up_sh", "down_sh", "gate_inp_sh",
                "logit_bias")


def synth_layer(g: Geom, seed: int, device="cuda", sigma: float = 0.02, logit_bias=None, stream=None) -> Dict:
    """A synthetic layer generated on the device (streams: 1 gate, 2 up, 3 down, 4 router, 5/6/7 shared
    gate/up/down, 8 shared gate_inp), bit-identical to the test oracle's host generators."""
    import torch
    L = lib()
    st = _stream(stream)
    H, F, Fs, E = g.n_embd, g.n_ff, g.n_ff_shared, g.n_expert

    def blocks(t, stream_id, n_values):
        buf = torch.empty(n_values // (64 if t == Q2_0 else 256) * (18 if t == Q2_0 else 82), dtype=torch.uint8,
                          device=device)
        _check(L.smoe_synth_blocks(t, seed, stream_id, n_values, sigma, buf.data_ptr(), st))
        return buf

    def bf16(stream_id, n):
        buf = torch.empty(n, dtype=torch.int16, device=device)
        _check(L.smoe_synth_bf16(seed, stream_id, n, sigma, buf.data_ptr(), st))
        return buf

    # the router is generated in f32 and kept in f32 (router_dtype 1) or stored as bf16 (the repo's contract)
    router = synth_normal(seed, 4, E * H, sigma, device=device, stream=stream) if g.router_dtype == ROUTER_F32 \
        else bf16(4, E * H)
    w = dict(gate_exps=blocks(g.w_type, 1, E * F * H), up_exps=blocks(g.w_type, 2, E * F * H),
             down_exps=blocks(g.w_type, 3, E * H * F), router=router)
    if g.sh_type >= 0:
        if any(t not in (Q2_0, IQ2_S) for t in g.shared_types()):
            raise ValueError("synth_layer generates Q2_0 and IQ2_S blocks only; upload other native types' blocks")
        tg, tu, td = g.shared_types()
        w.update(gate_sh=blocks(tg, 5, Fs * H), up_sh=blocks(tu, 6, Fs * H),
                 down_sh=blocks(td, 7, H * Fs), gate_inp_sh=bf16(8, H))
    if logit_bias is not None:
        w["logit_bias"] = logit_bias
    return w


def synth_normal(seed: int, stream_id: int, n: int, sigma: float = 1.0, device="cuda", stream=None):
    import torch
    out = torch.empty(n, dtype=torch.float32, device=device)
    _check(lib().smoe_synth_normal(seed, stream_id, n, sigma, out.data_ptr(), _stream(stream)))
    return out


def zipf_targets(n_expert: int, s: float, n_tokens: int, top_k: int):
    """Expected pairs per popularity rank r = 1 .. n_expert under Zipf(s): C * r^-s, capped at n_tokens (a token
    picks an expert at most once), with C such that the counts sum to n_tokens * top_k."""
    import numpy as np
    r = np.arange(1, n_expert + 1, dtype=np.float64)
    lo, hi = 0.0, float(n_tokens) * top_k * n_expert
    for _ in range(200):
        c = 0.5 * (lo + hi)
        if np.minimum(n_tokens, c * r ** -s).sum() < n_tokens * top_k:
            lo = c
        else:
            hi = c
    return np.minimum(n_tokens, 0.5 * (lo + hi) * r ** -s)


@functools.lru_cache(maxsize=8)
def _zipf_bias_cached(n_expert, s, seed, n_tokens, top_k, sigma, sims, iters):
    import numpy as np
    rng = np.random.default_rng(seed)
    rank_of = rng.permutation(n_expert)  # expert e has popularity rank rank_of[e]
    want = zipf_targets(n_expert, s, n_tokens, top_k) * (sims / n_tokens)
    tgt = np.clip(np.rint(want).astype(np.int64), 0, sims - 1)
    eps = rng.standard_normal((sims, n_expert)) * sigma
    b = np.log(want / want.mean()) * sigma
    cols = np.arange(n_expert)
    for _ in range(iters):
        z = eps + b
        head = -np.partition(-z, top_k, axis=1)[:, :top_k + 1]
        head.sort(axis=1)
        vk, vk1 = head[:, 1], head[:, 0]  # each token's k-th and (k+1)-th largest score
        # with the other experts' scores fixed, token t picks e iff b_e > (its k-th largest without e) - eps_te
        d = np.sort(np.where(z >= vk[:, None], vk1[:, None], vk[:, None]) - eps, axis=0)
        lo = np.where(tgt > 0, d[np.maximum(tgt - 1, 0), cols], d[0] - sigma)
        hi = np.where(tgt < sims, d[np.minimum(tgt, sims - 1), cols], d[-1] + sigma)
        b = b + 0.5 * (0.5 * (lo + hi) - b)
    return b[rank_of].astype(np.float32)


def zipf_bias(n_expert: int = 512, s: float = 1.2, seed: int = 1, n_tokens: int = 512, top_k: int = 10,
              n_embd: int = 2048, w_sigma: float = 0.02, sims: int = 4096, iters: int = 24):
    """Router logit bias of the prefill benchmark's routing: expert popularity follows
    Zipf(s) over a seeded rank permutation of the experts, i.e. the expected pairs of the rank-r expert are
    zipf_targets(...)[r-1] (hot experts take every token, many take none).  For x ~ N(0, 1) and router rows
    ~ N(0, w_sigma^2) a token's logits are close to independent N(0, sigma^2), sigma = w_sigma * sqrt(n_embd); the
    bias is fitted to that model by simulating `sims` tokens with fixed noise and solving, expert by expert, for
    the bias at which exactly its target share of the simulated tokens ranks it in their top k (damped
    fixed-point iterations).  Host-side and deterministic; an f32 numpy array of n_expert."""
    sigma = w_sigma * float(n_embd) ** 0.5
    return _zipf_bias_cached(n_expert, float(s), seed, n_tokens, top_k, sigma, sims, iters).copy()


def _weights_c(w: Dict) -> _Weights:
    return _Weights(*[_ptr(w.get(n)) for n in WEIGHT_NAMES])


class MoELayer:
    """One layer's MoE call: the FfnExec shape (metal/include/strata/metal/layer_exec.hpp:113-140) over
    smoe_forward.  Owns a workspace sized for `max_tokens`; weights stay the caller's tensors."""

    def __init__(self, g: Geom, weights: Dict, max_tokens: int, device="cuda"):
        import torch
        self.g = g
        self.w = weights
        self._gc = g.c()
        self._wc = _weights_c(weights)
        self.max_tokens = max_tokens
        self.ws_bytes = workspace_bytes(g, max_tokens)
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device=device)

    def forward(self, x, y=None, add_shared: bool = True, trace: bool = False, path: int = PATH_AUTO, stream=None,
                stages: bool = False):
        """y = MoE(x).  With `trace`, also returns the routing and the dispatch (logits, ids, weights, counts,
        offsets, perm, slot, sgate); with `stages` as well, the expert stages (xq, hq: q8_1 blocks of x and of each
        pair's h on the decode path; egate, eup: each pair's gate and up dots; sgu, shq: the shared expert's gate and
        up dots ([2][T][n_ff_shared]) and the q8_1 blocks of its h; parts, shared: each pair's expert output and the
        shared expert's, by dispatch position) and the prefill path's fp16 `overflow` mask -- the decode path then
        runs its unfused kernels."""
        import torch
        if x.dim() != 2:
            raise SmoeError(-1, f"x must be (tokens, {self.g.n_embd}), got {tuple(x.shape)}")
        T = x.shape[0]
        _need(x, "x", torch.float32, shape=(T, self.g.n_embd))
        if T > self.max_tokens:
            raise SmoeError(-2, f"{T} tokens exceed the workspace's {self.max_tokens}")
        if y is None:
            y = torch.empty_like(x)
        _need(y, "y", torch.float32, numel=T * self.g.n_embd)
        tr = None
        out = {}
        if trace:
            E, K, dev = self.g.n_expert, self.g.top_k, x.device
            out = dict(logits=torch.empty((T, E), dtype=torch.float32, device=dev),
                       ids=torch.empty((T, K), dtype=torch.int32, device=dev),
                       weights=torch.empty((T, K), dtype=torch.float32, device=dev),
                       counts=torch.empty(E, dtype=torch.int32, device=dev),
                       offsets=torch.empty(E + 1, dtype=torch.int32, device=dev),
                       perm=torch.empty(T * K, dtype=torch.int32, device=dev),
                       slot=torch.empty(T * K, dtype=torch.int32, device=dev),
                       sgate=torch.empty(T, dtype=torch.float32, device=dev))
            names = ["logits", "ids", "weights", "counts", "offsets", "perm", "slot", "sgate"]
            if stages:
                H, F, Fs = self.g.n_embd, self.g.n_ff, max(self.g.n_ff_shared, 32)
                out.update(xq=torch.empty((T, H // 32 * 36), dtype=torch.uint8, device=dev),
                           hq=torch.empty((T * K, F // 32 * 36), dtype=torch.uint8, device=dev),
                           parts=torch.empty((T * K, H), dtype=torch.float32, device=dev),
                           shared=torch.empty((T, H), dtype=torch.float32, device=dev),
                           overflow=torch.full((1,), -1, dtype=torch.int32, device=dev),
                           egate=torch.empty((T * K, F), dtype=torch.float32, device=dev),
                           eup=torch.empty((T * K, F), dtype=torch.float32, device=dev),
                           sgu=torch.empty((2, T, Fs), dtype=torch.float32, device=dev),
                           shq=torch.empty((T, Fs // 32 * 36), dtype=torch.uint8, device=dev))
            tr = _Trace(*[out[n].data_ptr() for n in names], None,
                        *[out[n].data_ptr() if stages else None
                          for n in ("xq", "hq", "parts", "shared", "overflow", "egate", "eup", "sgu", "shq")])
        _check(lib().smoe_forward_path(C.byref(self._gc), C.byref(self._wc), x.data_ptr(), T, y.data_ptr(),
                                       int(add_shared), self.ws.data_ptr(), self.ws_bytes,
                                       None if tr is None else C.byref(tr), path, _stream(stream)))
        return (y, out) if trace else y

    def status(self, stream=None):
        """The status mask of the last call on this layer's workspace (smoe_forward_status), as a device int32
        tensor: 0, or STATUS_X_FP16 | STATUS_H_FP16 (the prefill path's fp16 operand limits) | STATUS_WAIT (a
        fused decode launch's wait gave up; its rows are NaN)."""
        import torch
        out = torch.full((1,), -1, dtype=torch.int32, device=self.ws.device)
        _check(lib().smoe_forward_status(self.ws.data_ptr(), out.data_ptr(), _stream(stream)))
        return out

    def forward_residual(self, x_prev, r_prev, x, y=None, eps: float = 1e-6, add_shared: bool = True, stream=None):
        """The stack junction fused into this layer's call: x = RMSNorm(x_prev + r_prev) (written to `x`), then
        y = MoE(x) (smoe_forward_residual).  `x` must not overlap x_prev, r_prev or y; y may be r_prev."""
        import torch
        if x.dim() != 2:
            raise SmoeError(-1, f"x must be (tokens, {self.g.n_embd}), got {tuple(x.shape)}")
        T = x.shape[0]
        shape = (T, self.g.n_embd)
        for t, name in ((x_prev, "x_prev"), (r_prev, "r_prev"), (x, "x")):
            _need(t, name, torch.float32, shape=shape)
        if T > self.max_tokens:
            raise SmoeError(-2, f"{T} tokens exceed the workspace's {self.max_tokens}")
        if y is None:
            y = torch.empty_like(x)
        _need(y, "y", torch.float32, numel=T * self.g.n_embd)
        _check(lib().smoe_forward_residual(C.byref(self._gc), C.byref(self._wc), x_prev.data_ptr(), r_prev.data_ptr(),
                                           eps, x.data_ptr(), T, y.data_ptr(), int(add_shared), self.ws.data_ptr(),
                                           self.ws_bytes, None, _stream(stream)))
        return y

    __call__ = forward


# ------------------------------------------------------------------------------------------------ layer ends

class HyperConnection:
    """The gated-residual ends of the layer call (smoe_hc_read / smoe_hc_write), the gr_read / gr_write pair of
    FfnExec::run (metal/include/strata/metal/gr.hpp:44-48).  `norm` is [hc * n_embd] f32 (the stored 1 + w);
    `down` [hc_lr][hc * n_embd], `up` [hc * n_embd][hc_lr] and `inject` [hc][hc * n_embd] are bf16 bits (int16)."""

    def __init__(self, n_embd: int, hc: int, hc_lr: int, norm, down, up, inject, eps: float = 1e-6):
        import torch
        hd = hc * n_embd
        _need(norm, "norm", torch.float32, numel=hd)
        for t, name, k in ((down, "down", hc_lr * hd), (up, "up", hd * hc_lr), (inject, "inject", hc * hd)):
            _need(t, name, torch.int16, numel=k)
        self.n_embd, self.hc, self.hc_lr, self.eps = n_embd, hc, hc_lr, eps
        self.tensors = (norm, down, up, inject)
        self._c = _Hc(hc, hc_lr, eps, norm.data_ptr(), down.data_ptr(), up.data_ptr(), inject.data_ptr())
        self._ws = None

    def _stream_tensor(self, R, name="R"):
        import torch
        if R.dim() != 3 or tuple(R.shape[1:]) != (self.hc, self.n_embd):
            raise SmoeError(-1, f"{name} must be (tokens, {self.hc}, {self.n_embd}), got {tuple(R.shape)}")
        return _need(R, name, torch.float32)

    def read(self, R, mixed=None, inject=None, stream=None):
        """mixed [T][n_embd], inject [T][hc] of the streams R [T][hc][n_embd]."""
        import torch
        R = self._stream_tensor(R)
        T = R.shape[0]
        if mixed is None:
            mixed = torch.empty((T, self.n_embd), dtype=torch.float32, device=R.device)
        if inject is None:
            inject = torch.empty((T, self.hc), dtype=torch.float32, device=R.device)
        _need(mixed, "mixed", torch.float32, numel=T * self.n_embd)
        _need(inject, "inject", torch.float32, numel=T * self.hc)
        n = lib().smoe_hc_read_workspace_bytes(C.byref(self._c), self.n_embd, max(T, 1))
        if n == 0:
            raise SmoeError(-1, lib().smoe_last_error().decode() or "bad hyper-connection shape")
        if self._ws is None or self._ws.numel() < n:
            self._ws = torch.empty(n, dtype=torch.uint8, device=R.device)
        _check(lib().smoe_hc_read(C.byref(self._c), self.n_embd, R.data_ptr(), T, mixed.data_ptr(), inject.data_ptr(),
                                  self._ws.data_ptr(), self._ws.numel(), _stream(stream)))
        return mixed, inject

    def write(self, R, y, inject, out=None, stream=None):
        """out = R + y * 2 sigmoid(inject / hc) on every stream; `out` may be R."""
        import torch
        R = self._stream_tensor(R)
        T = R.shape[0]
        _need(y, "y", torch.float32, numel=T * self.n_embd)
        _need(inject, "inject", torch.float32, numel=T * self.hc)
        if out is None:
            out = torch.empty_like(R)
        _need(out, "out", torch.float32, numel=R.numel())
        _check(lib().smoe_hc_write(C.byref(self._c), self.n_embd, R.data_ptr(), y.data_ptr(), inject.data_ptr(), T,
                                   out.data_ptr(), _stream(stream)))
        return out


class FfnLayer:
    """FfnExec::run(residual, out, add_shared, trace) (metal/include/strata/metal/layer_exec.hpp:135-137): gr_read of
    the residual streams, the MoE block, gr_write back onto the streams, in one smoe_ffn_run call.  Owns a workspace
    sized for `max_tokens`."""

    def __init__(self, g: Geom, weights: Dict, hc: HyperConnection, max_tokens: int, device="cuda"):
        import torch
        if hc.n_embd != g.n_embd:
            raise SmoeError(-1, f"hyper connection width {hc.n_embd} != n_embd {g.n_embd}")
        self.g, self.w, self.hc = g, weights, hc
        self._gc, self._wc = g.c(), _weights_c(weights)
        self.max_tokens = max_tokens
        self.ws_bytes = lib().smoe_ffn_workspace_bytes(C.byref(self._gc), C.byref(hc._c), max_tokens)
        if self.ws_bytes == 0:
            raise SmoeError(-1, lib().smoe_last_error().decode() or "bad geometry")
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device=device)

    def run(self, residual, out=None, add_shared: bool = True, stream=None):
        import torch
        R = self.hc._stream_tensor(residual, "residual")
        T = R.shape[0]
        if T > self.max_tokens:
            raise SmoeError(-2, f"{T} tokens exceed the workspace's {self.max_tokens}")
        if out is None:
            out = torch.empty_like(R)
        _need(out, "out", torch.float32, numel=R.numel())
        _check(lib().smoe_ffn_run(C.byref(self._gc), C.byref(self._wc), C.byref(self.hc._c), R.data_ptr(), T,
                                  out.data_ptr(), int(add_shared), self.ws.data_ptr(), self.ws_bytes, None,
                                  _stream(stream)))
        return out

    __call__ = run


# ------------------------------------------------------------------------------------------------ stages

def router_topk(logits, k: int, stream=None):
    import torch
    if logits.dim() != 2:
        raise SmoeError(-1, "logits must be (tokens, experts)")
    T, E = logits.shape
    _need(logits, "logits", torch.float32)
    ids = torch.empty((T, k), dtype=torch.int32, device=logits.device)
    w = torch.empty((T, k), dtype=torch.float32, device=logits.device)
    _check(lib().smoe_router_topk(logits.data_ptr(), T, E, k, ids.data_ptr(), w.data_ptr(), _stream(stream)))
    return ids, w


def router_margin(logits, k: int, stream=None):
    """The router-margin diagnostic (smoe_router_margin): stats (T, 4) = (p_k - p_k1, logit gap, p_k, p_k1) and
    ids (T, 2) = (id_k, id_k1) of the k-th and (k+1)-th experts by softmax probability."""
    import torch
    if logits.dim() != 2:
        raise SmoeError(-1, "logits must be (tokens, n_expert)")
    _need(logits, "logits", torch.float32)
    T, E = logits.shape
    stats = torch.empty((T, 4), dtype=torch.float32, device=logits.device)
    ids = torch.empty((T, 2), dtype=torch.int32, device=logits.device)
    _check(lib().smoe_router_margin(logits.data_ptr(), T, E, k, stats.data_ptr(), ids.data_ptr(), _stream(stream)))
    return stats, ids


def f32_to_bf16(x, stream=None):
    import torch
    _need(x, "x", torch.float32)
    y = torch.empty(x.shape, dtype=torch.int16, device=x.device)
    _check(lib().smoe_f32_to_bf16(x.data_ptr(), x.numel(), y.data_ptr(), _stream(stream)))
    return y


def bf16_gemv(x_bf16, w_bf16, n_in: int, n_out: int, stream=None):
    import torch
    _need(x_bf16, "x_bf16", torch.int16)
    _need(w_bf16, "w_bf16", torch.int16, numel=n_in * n_out)
    if n_in <= 0 or x_bf16.numel() % n_in:
        raise SmoeError(-1, f"x_bf16 holds {x_bf16.numel()} values, not whole rows of {n_in}")
    n_tok = x_bf16.numel() // n_in
    y = torch.empty((n_tok, n_out), dtype=torch.float32, device=x_bf16.device)
    _check(lib().smoe_bf16_gemv(x_bf16.data_ptr(), w_bf16.data_ptr(), y.data_ptr(), n_in, n_out, n_tok,
                                _stream(stream)))
    return y


def quantize_q8_1(x, stream=None):
    import torch
    _need(x, "x", torch.float32)
    y = torch.empty(x.numel() // 32 * 36, dtype=torch.uint8, device=x.device)
    _check(lib().smoe_quantize_q8_1(x.data_ptr(), x.numel(), y.data_ptr(), _stream(stream)))
    return y


def mmvq(wtype: int, w, x_q8, n_in: int, n_out: int, n_col: int = 1, byte_off: int = 0, stream=None):
    import torch
    _need(w, "w", torch.uint8, numel=byte_off + n_out * row_bytes(wtype, n_in))
    _need(x_q8, "x_q8", torch.uint8, numel=n_col * (n_in // 32) * 36)
    y = torch.empty((n_col, n_out), dtype=torch.float32, device=w.device)
    _check(lib().smoe_mmvq(wtype, w.data_ptr(), byte_off, x_q8.data_ptr(), n_in, n_out, n_col, y.data_ptr(),
                           _stream(stream)))
    return y


def expert(blob, x_q8, gu_type: int, d_type: int, n_embd: int, n_ff: int, n_tok: int, stream=None):
    """One expert's FFN on a [gate | up | down] blob (smoe_expert; the reference's iq_expert)."""
    import torch
    _need(blob, "blob", torch.uint8)
    _need(x_q8, "x_q8", torch.uint8, numel=n_tok * (n_embd // 32) * 36)
    L = lib()
    scratch = torch.empty(L.smoe_expert_scratch_bytes(n_embd, n_ff, n_tok) + 256, dtype=torch.uint8,
                          device=blob.device)
    base = (scratch.data_ptr() + 255) & ~255
    y = torch.empty((n_tok, n_embd), dtype=torch.float32, device=blob.device)
    _check(L.smoe_expert(blob.data_ptr(), blob.numel(), x_q8.data_ptr(), gu_type, d_type, n_embd, n_ff, n_tok,
                         y.data_ptr(), base, scratch.numel() - (base - scratch.data_ptr()), _stream(stream)))
    return y


def residual_rmsnorm(x, r=None, eps: float = 1e-6, out=None, stream=None):
    """RMSNorm(x + r) row by row with unit weight (smoe_residual_rmsnorm); `out` may be `x`."""
    import torch
    _need(x, "x", torch.float32)
    n = x.shape[-1]
    if r is not None:
        _need(r, "r", torch.float32, shape=x.shape)
    out = torch.empty_like(x) if out is None else out
    _need(out, "out", torch.float32, shape=x.shape)
    _check(lib().smoe_residual_rmsnorm(x.data_ptr(), _ptr(r), x.numel() // n, n, eps, out.data_ptr(), _stream(stream)))
    return out


def swiglu_q8(gate, up, stream=None):
    import torch
    _need(gate, "gate", torch.float32)
    _need(up, "up", torch.float32, shape=gate.shape)
    y = torch.empty(gate.numel() // 32 * 36, dtype=torch.uint8, device=gate.device)
    _check(lib().smoe_swiglu_q8(gate.data_ptr(), up.data_ptr(), gate.numel(), y.data_ptr(), _stream(stream)))
    return y


def combine(parts, weights, shared=None, stream=None):
    import torch
    if parts.dim() != 2:
        raise SmoeError(-1, "parts must be (k, n_embd)")
    _need(parts, "parts", torch.float32)
    k, n = parts.shape
    _need(weights, "weights", torch.float32, numel=k)
    if shared is not None:
        _need(shared, "shared", torch.float32, numel=n)
    y = torch.empty(n, dtype=torch.float32, device=parts.device)
    _check(lib().smoe_combine(parts.data_ptr(), weights.data_ptr(), _ptr(shared), y.data_ptr(), n, k,
                              _stream(stream)))
    return y


def dispatch(ids, n_expert: int, stream=None):
    import torch
    if ids.dim() != 2:
        raise SmoeError(-1, "ids must be (tokens, k)")
    _need(ids, "ids", torch.int32)
    T, k = ids.shape
    dev = ids.device
    counts = torch.empty(n_expert, dtype=torch.int32, device=dev)
    offsets = torch.empty(n_expert + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(T * k, dtype=torch.int32, device=dev)
    slot = torch.empty(T * k, dtype=torch.int32, device=dev)
    _check(lib().smoe_dispatch(ids.data_ptr(), T, k, n_expert, counts.data_ptr(), offsets.data_ptr(),
                               perm.data_ptr(), slot.data_ptr(), _stream(stream)))
    return counts, offsets, perm, slot


# ------------------------------------------------------------------------------------------------ GGUF models

class _TensorInfo(C.Structure):
    _fields_ = [("type", C.c_int32), ("n_dims", C.c_int32), ("shard", C.c_int32), ("reserved", C.c_int32),
                ("ne", C.c_uint64 * 4), ("bytes", C.c_uint64), ("file_offset", C.c_uint64), ("host", C.c_void_p)]


class _LayerPlan(C.Structure):
    _fields_ = [("geom", _Geom), ("hc", _Hc), ("device_bytes", C.c_size_t), ("off", C.c_size_t * 12),
                ("layer", C.c_int32), ("with_shared", C.c_int32)]


@dataclass
class TensorInfo:
    name: str
    type: int
    shape: tuple           # GGUF order: shape[0] is a row
    shard: int
    bytes: int
    file_offset: int


class Model:
    """A GGUF v3 model on the host (smoe_model_*: every shard of a split model, mapped read-only), its tensors by
    name, its metadata, and one layer's MoE tensors loaded into device memory (smoe_layer_plan_for /
    smoe_layer_upload, the tensor side of the reference's FfnExec::load)."""

    def __init__(self, path: str):
        self._h = C.c_void_p()
        _check(lib().smoe_model_open(path.encode(), C.byref(self._h)))

    def close(self):
        if self._h:
            lib().smoe_model_close(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def n_shards(self) -> int:
        return int(lib().smoe_model_n_shards(self._h))

    def _info(self, name: str, ti: _TensorInfo) -> TensorInfo:
        return TensorInfo(name, ti.type, tuple(int(ti.ne[d]) for d in range(ti.n_dims)), ti.shard, int(ti.bytes),
                          int(ti.file_offset))

    def tensors(self):
        out = []
        for i in range(int(lib().smoe_model_n_tensors(self._h))):
            buf = C.create_string_buffer(4096)
            ti = _TensorInfo()
            _check(lib().smoe_model_tensor_at(self._h, i, buf, 4096, C.byref(ti)))
            out.append(self._info(buf.value.decode(), ti))
        return out

    def tensor(self, name: str) -> TensorInfo:
        ti = _TensorInfo()
        _check(lib().smoe_model_tensor(self._h, name.encode(), C.byref(ti)))
        return self._info(name, ti)

    def tensor_bytes(self, name: str) -> bytes:
        """The payload as the mapping holds it (a copy)."""
        ti = _TensorInfo()
        _check(lib().smoe_model_tensor(self._h, name.encode(), C.byref(ti)))
        return C.string_at(ti.host, ti.bytes)

    def meta_u64(self, key: str) -> int:
        v = C.c_uint64()
        _check(lib().smoe_model_meta_u64(self._h, key.encode(), C.byref(v)))
        return int(v.value)

    def meta_str(self, key: str) -> str:
        buf = C.create_string_buffer(1 << 16)
        _check(lib().smoe_model_meta_str(self._h, key.encode(), buf, 1 << 16))
        return buf.value.decode()

    def plan(self, layer: int, top_k: int = 0, with_shared: bool = True) -> _LayerPlan:
        p = _LayerPlan()
        _check(lib().smoe_layer_plan_for(self._h, layer, top_k, int(with_shared), C.byref(p)))
        return p

    def load_layer(self, layer: int, top_k: int = 0, with_shared: bool = True, with_hc: bool = False,
                   device="cuda", stream=None):
        """(Geom, weights dict of device tensors, HyperConnection or None) of one layer; the weights are views of
        one device buffer the returned dict also keeps (key "_buffer")."""
        import torch
        p = self.plan(layer, top_k, with_shared)
        buf = torch.empty(p.device_bytes + 256, dtype=torch.uint8, device=device)
        base = (buf.data_ptr() + 255) & ~255
        w, hc = _Weights(), _Hc()
        _check(lib().smoe_layer_upload(self._h, C.byref(p), base, p.device_bytes, C.byref(w),
                                       C.byref(hc) if with_hc else None, _stream(stream)))
        gc = p.geom
        g = Geom(gc.n_embd, gc.n_ff, gc.n_ff_shared, gc.n_expert, gc.top_k, gc.w_type, gc.sh_type, gc.router_dtype,
                 gc.sh_gate_type, gc.sh_up_type, gc.sh_down_type)

        def view(ptr, nbytes):
            o = ptr - buf.data_ptr()
            return buf[o:o + nbytes]

        H, F, E, Fs = g.n_embd, g.n_ff, g.n_expert, g.n_ff_shared
        sizes = dict(gate_exps=E * F * row_bytes(g.w_type, H), up_exps=E * F * row_bytes(g.w_type, H),
                     down_exps=E * H * row_bytes(g.w_type, F),
                     router=E * H * (4 if g.router_dtype == ROUTER_F32 else 2))
        weights = {n: view(getattr(w, n), sizes[n]) for n in sizes}
        if with_shared:
            weights.update(gate_sh=view(w.gate_sh, Fs * row_bytes(g.sh_gate_type, H)),
                           up_sh=view(w.up_sh, Fs * row_bytes(g.sh_up_type, H)),
                           down_sh=view(w.down_sh, H * row_bytes(g.sh_down_type, Fs)),
                           gate_inp_sh=view(w.gate_inp_sh, H * 2))
        weights["_buffer"] = buf
        hcx = None
        if with_hc:
            hd = hc.hc * H
            hcx = HyperConnection(H, hc.hc, hc.hc_lr, view(hc.norm, hd * 4).view(torch.float32),
                                  view(hc.down, hc.hc_lr * hd * 2).view(torch.int16),
                                  view(hc.up, hd * hc.hc_lr * 2).view(torch.int16),
                                  view(hc.inject, hc.hc * hd * 2).view(torch.int16), eps=float(hc.eps))
        return g, weights, hcx


# ------------------------------------------------------------------------------------------------ expert tier

def expert_blob_bytes(g: Geom) -> int:
    """Bytes of one routed expert's blob [gate rows | up rows | down rows] (smoe_expert_blob_bytes)."""
    n = int(lib().smoe_expert_blob_bytes(C.byref(g.c())))
    if n == 0:
        raise SmoeError(-1, lib().smoe_last_error().decode())
    return n


def pack_expert(g: Geom, weights: Dict, expert: int, blob, stream=None):
    """Copies expert `expert`'s rows from the planes in `weights` into `blob` (uint8, expert_blob_bytes)."""
    import torch
    _need(blob, "blob", torch.uint8, numel=expert_blob_bytes(g))
    _check(lib().smoe_expert_pack(C.byref(g.c()), C.byref(_weights_c(weights)), expert, blob.data_ptr(),
                                  _stream(stream)))
    return blob


def expert_table(ptrs, device="cuda"):
    """A device table of one blob address per expert (0: not held) from a list of tensors or None."""
    import torch
    a = [0 if t is None else t.data_ptr() for t in ptrs]
    return torch.tensor(a, dtype=torch.int64, device=device)


def expert_group(ids, k_per_tok: int, n_expert: int, table, stream=None) -> Dict:
    """The hit/miss split of the routed entries `ids` (int32, T * k_per_tok) by the expert table (int64 device
    addresses, 0 = not held), on the device (smoe_expert_group): grp_ptr, grp_expert, grp_start, ent_dst,
    ent_tok, miss_dst and counts {groups, hits, misses, 0}."""
    import torch
    _need(ids, "ids", torch.int32)
    _need(table, "table", torch.int64, numel=n_expert)
    n = ids.numel()
    G = max(1, min(n, n_expert))
    dev = ids.device
    out = dict(grp_ptr=torch.zeros(G, dtype=torch.int64, device=dev),
               grp_expert=torch.full((G,), -1, dtype=torch.int32, device=dev),
               grp_start=torch.zeros(G + 1, dtype=torch.int32, device=dev),
               ent_dst=torch.full((max(n, 1),), -1, dtype=torch.int32, device=dev),
               ent_tok=torch.full((max(n, 1),), -1, dtype=torch.int32, device=dev),
               miss_dst=torch.full((max(n, 1),), -1, dtype=torch.int32, device=dev),
               counts=torch.zeros(4, dtype=torch.int32, device=dev))
    _check(lib().smoe_expert_group(ids.data_ptr(), n, k_per_tok, n_expert, table.data_ptr(),
                                   out["grp_ptr"].data_ptr(), out["grp_start"].data_ptr(),
                                   out["grp_expert"].data_ptr(), out["ent_dst"].data_ptr(), out["ent_tok"].data_ptr(),
                                   out["miss_dst"].data_ptr(), out["counts"].data_ptr(), _stream(stream)))
    return out


def expert_grouped(g: Geom, groups: Dict, x_q8, n_tokens: int, out, cap_groups: int = None, cap_entries: int = None,
                   stream=None):
    """Grouped expert evaluation (smoe_expert_grouped) over the lists in `groups` (expert_group's keys): each
    entry's expert output row written to out[ent_dst] (out: (rows, n_embd) f32)."""
    import torch
    cg = groups["grp_ptr"].numel() if cap_groups is None else cap_groups
    ce = groups["ent_dst"].numel() if cap_entries is None else cap_entries
    # the kernels read the lists up to the caps: every list must hold them
    lists = (("grp_ptr", torch.int64, cg), ("grp_start", torch.int32, cg + 1), ("ent_dst", torch.int32, ce),
             ("ent_tok", torch.int32, ce), ("counts", torch.int32, 2))
    for key, _, n in lists:
        if groups[key].numel() < n:
            raise SmoeError(-2, f"{key} has {groups[key].numel()} elements, needs {n}")
    if out.dim() != 2 or out.shape[1] != g.n_embd:
        raise SmoeError(-2, f"out has shape {tuple(out.shape)}, needs (rows, {g.n_embd})")
    for key, dtype, n in lists:
        _need(groups[key], key, dtype, numel=n)
    _need(x_q8, "x_q8", torch.uint8, numel=n_tokens * (g.n_embd // 32) * 36)
    _need(out, "out", torch.float32)
    nb = int(lib().smoe_expert_grouped_workspace_bytes(C.byref(g.c()), n_tokens, cg, ce))
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device=out.device)
    _check(lib().smoe_expert_grouped(C.byref(g.c()), groups["grp_ptr"].data_ptr(), groups["grp_start"].data_ptr(),
                                     groups["ent_dst"].data_ptr(), groups["ent_tok"].data_ptr(),
                                     groups["counts"].data_ptr(), cg, ce, x_q8.data_ptr(), n_tokens, out.data_ptr(),
                                     out.shape[0], ws.data_ptr(), nb, _stream(stream)))
    return out


class VerifyWindow:
    """The verify window with the hit/miss split (smoe_verify_begin / smoe_verify_end): `begin` routes the tokens,
    computes the hits from the expert table and the shared expert into rows, and returns the misses for the caller
    to fill; `end` combines the rows into y."""

    def __init__(self, g: Geom, weights: Dict, max_tokens: int, device="cuda"):
        import torch
        self.g, self.w = g, weights
        self._gc, self._wc = g.c(), _weights_c(weights)
        self.ws_bytes = int(lib().smoe_verify_workspace_bytes(C.byref(self._gc), max_tokens))
        if self.ws_bytes == 0:
            raise SmoeError(-1, f"verify window refused for {max_tokens} tokens: {lib().smoe_last_error().decode()}")
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device=device)
        self.max_tokens = max_tokens

    def begin(self, x, table, stream=None) -> Dict:
        import torch
        _need(x, "x", torch.float32)
        T, H, K = x.shape[0], self.g.n_embd, self.g.top_k
        if x.dim() != 2 or x.shape[1] != H:
            raise SmoeError(-2, f"x has shape {tuple(x.shape)}, needs (tokens, {H})")
        if T > self.max_tokens:
            raise SmoeError(-1, f"{T} tokens exceed the window's {self.max_tokens}")
        _need(table, "table", torch.int64, numel=self.g.n_expert)
        dev = x.device
        r = dict(rows=torch.zeros((T * K + T, H), dtype=torch.float32, device=dev),
                 ids=torch.empty((T, K), dtype=torch.int32, device=dev),
                 weights=torch.empty((T, K), dtype=torch.float32, device=dev),
                 miss_dst=torch.full((max(T * K, 1),), -1, dtype=torch.int32, device=dev),
                 counts=torch.zeros(4, dtype=torch.int32, device=dev))
        _check(lib().smoe_verify_begin(C.byref(self._gc), C.byref(self._wc), table.data_ptr(), x.data_ptr(), T,
                                       r["rows"].data_ptr(), r["ids"].data_ptr(), r["weights"].data_ptr(),
                                       r["miss_dst"].data_ptr(), r["counts"].data_ptr(), self.ws.data_ptr(),
                                       self.ws_bytes, _stream(stream)))
        return r

    def end(self, r: Dict, add_shared: bool = True, y=None, stream=None):
        import torch
        T, H, K = r["ids"].shape[0], self.g.n_embd, self.g.top_k
        _need(r["rows"], "rows", torch.float32, numel=(T * K + T) * H)
        _need(r["weights"], "weights", torch.float32, numel=T * K)
        if y is None:
            y = torch.empty((T, H), dtype=torch.float32, device=r["rows"].device)
        _need(y, "y", torch.float32, numel=T * H)
        _check(lib().smoe_verify_end(C.byref(self._gc), T, r["rows"].data_ptr(), r["weights"].data_ptr(),
                                     int(add_shared), y.data_ptr(), self.ws.data_ptr(), self.ws_bytes,
                                     _stream(stream)))
        return y

