#!/usr/bin/env python
"""bench.py - MoE-layer throughput of the MI355X quantized MoE block (BASELINE.json's metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one MoE layer call (router, top-k, dispatch, expert products, shared expert, combine) on one batch of
synthetic tokens.  The headline workload is BASELINE.json configs[0]: one Qwen3-Next-style layer (H 2048, 512 Q2_0
experts + 1 shared, top-10, FF 512) decoding one token.  `--layers` (default 48, ~21.7 GB) distinct layers are
resident in HBM and consecutive steps walk through them, each with its own token; the K timed steps are one
captured HIP graph replay, and a 1 GiB read between replays empties the 256 MB Infinity Cache (MALL) of the layers'
bytes, so every step reads its layer's bytes from HBM.  Per-stage kernel durations come from HIP events recorded on the launch
stream between the kernels of an eager pass of the same steps (also after a flush).  The JSON line's `roofline` is
the dominant decode kernel's; `roofline_prefill_512` is the prefill GEMM's (configs[2], the metric's second half).
`extra` holds decode batch 16, prefill 512 with Zipf(1.2) routing, IQ2_S batch 64
(configs[3]) and the 48-layer stack.  The CPU baseline is the test oracle's C restatement of the
reference's host path organised as the reference's CPU pool (kind "port"), built for and timed on this host.
Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer tok/s + achieved HBM GB/s vs peak, decode b=1 and prefill 512"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA
FLUSH_BYTES = 1 << 30      # four times the MALL


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=96)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--no-extra", action="store_true", help="only the headline (decode b=1)")
    ap.add_argument("--prefill-layers", type=int, default=8)
    ap.add_argument("--prefill-steps", type=int, default=24)
    ap.add_argument("--iq2-layers", type=int, default=8)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB five times (the reference kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters to bytes), then exit")
    ap.add_argument("--only", choices=("b1", "b16", "prefill", "iq2", "stack"), default=None,
                    help="measure only this workload (for a profiler run); prints its summary, no JSON line")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--flush", choices=("read", "write"), default="read",
                    help="how the 1 GiB cache flush between timed passes touches its buffer")
    ap.add_argument("--stack-prefill", type=int, default=4096, help="prefill tokens of the 48-layer stack")
    ap.add_argument("--stack-decode", type=int, default=64, help="decode steps of the 48-layer stack")
    ap.add_argument("--cpu-seconds", type=float, default=3.0, help="CPU baseline seconds per (workload, threads)")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def source_digest():
    """sha256 of the library's sources: a profile summary applies to the build whose digest it records."""
    h = hashlib.sha256()
    d = os.path.join(ROOT, "stratametal_amd", "csrc")
    for f in sorted(os.listdir(d)):
        h.update(f.encode())
        h.update(open(os.path.join(d, f), "rb").read())
    return h.hexdigest()[:16]


def profile_record(name, kernel):
    """A committed counter summary (profiles/<name>.json) for `kernel`, if it was taken from the current sources."""
    p = os.path.join(ROOT, "profiles", name + ".json")
    if not os.path.exists(p):
        return None
    rec = json.load(open(p))
    if rec.get("source_digest") != source_digest() or not rec.get("kernel", "").startswith(kernel):
        return None
    return rec


class Stack:
    """`n_layers` synthetic layers resident on the device, one workspace, a graph per token count."""

    def __init__(self, S, torch, g, n_layers, seed, max_tokens, logit_bias=None, layers=None):
        self.S, self.torch, self.g, self.seed, self.max_tokens = S, torch, g, seed, max_tokens
        self.layers = layers if layers is not None else [S.synth_layer(g, seed + l, logit_bias=logit_bias)
                                                         for l in range(n_layers)]
        self.wc = [S._weights_c(w) for w in self.layers]
        self.gc = g.c()
        self.ws_bytes = S.workspace_bytes(g, max_tokens)
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()

    def with_f32_router(self):
        """The same layers with the literal configs[0]'s f32 router (router_dtype 1): the expert tensors are shared,
        each router is the f32 the bf16 one was rounded from (synth_layer's stream 4)."""
        S, g = self.S, self.g
        g32 = S.Geom(**dict(vars(g), router_dtype=S.ROUTER_F32))
        layers = [dict(w, router=S.synth_normal(self.seed + l, 4, g.n_expert * g.n_embd, 0.02))
                  for l, w in enumerate(self.layers)]
        return Stack(S, self.torch, g32, len(layers), self.seed, self.max_tokens, layers=layers)

    def inputs(self, T, seed):
        S, g = self.S, self.g
        xs = S.synth_normal(seed, 100 + T, len(self.layers) * T * g.n_embd).view(len(self.layers), T, g.n_embd)
        return xs, self.torch.empty_like(xs)

    def call(self, l, x, y, T, trace=None):
        import ctypes as C
        S = self.S
        st = S.lib().smoe_forward(C.byref(self.gc), C.byref(self.wc[l]), x.data_ptr(), T, y.data_ptr(), 1,
                                  self.ws.data_ptr(), self.ws_bytes, None if trace is None else C.byref(trace),
                                  S._stream())
        S._check(st)


class HipEvents:
    """Raw hipEvent_t handles (timing enabled) from the HIP runtime, for the library's stage-event hook."""

    def __init__(self):
        import ctypes as C
        self.C = C
        self.hip = C.CDLL("libamdhip64.so")
        self.hip.hipEventCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]

    def create(self, n):
        out = []
        for _ in range(n):
            ev = self.C.c_void_p()
            # no system-scope fence at record (no cache writeback between kernels): the events only time kernels
            if self.hip.hipEventCreateWithFlags(self.C.byref(ev), 0x20000000) != 0:  # hipEventDisableSystemFence
                raise RuntimeError("hipEventCreateWithFlags failed")
            out.append(ev.value)
        return out

    def elapsed_ms(self, a, b):
        ms = self.C.c_float()
        if self.hip.hipEventElapsedTime(self.C.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value


class Flush:
    """A 1 GiB buffer read (or, with --flush write, rewritten) between timed passes, so that no layer's bytes are
    left in the MALL or L2.  Reading leaves clean lines behind: a rewrite leaves the MALL full of dirty lines whose
    write-back then competes with the timed steps' reads."""

    def __init__(self, torch, mode="read"):
        self.buf = torch.zeros(FLUSH_BYTES // 4, dtype=torch.float32, device="cuda")
        self.mode = mode

    def __call__(self):
        if self.mode == "write":
            self.buf.add_(1.0)
        else:
            self.sink = self.buf.sum()


def measure(S, torch, stack, T, steps, warmup, seed, flush):
    """Time `steps` layer calls at T tokens (one graph replay, caches flushed first); return the wall time, the
    replay's event time, per-stage durations of an eager pass with stage events, and the touched experts."""
    g = stack.g
    L = len(stack.layers)
    xs, ys = stack.inputs(T, seed)
    E = g.n_expert
    counts = torch.zeros((steps, E), dtype=torch.int32, device="cuda")
    he = HipEvents()
    events = [he.create(S.STAGE_EVENTS) for _ in range(steps)]
    evp = [(S.C.c_void_p * S.STAGE_EVENTS)(*evs) for evs in events]
    traces = [S._Trace(None, None, None, counts[s].data_ptr(), None, None, None, None,
                       S.C.cast(evp[s], S.C.c_void_p)) for s in range(steps)]
    for s in range(warmup):  # eager warmup (also loads the code objects)
        stack.call(s % L, xs[s % L], ys[s % L], T)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for s in range(steps):
                tr = S._Trace(None, None, None, counts[s].data_ptr(), None, None, None, None, None)
                stack.call(s % L, xs[s % L], ys[s % L], T, tr)
    torch.cuda.synchronize()
    graph.replay()  # untimed: code and graph resident
    flush()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    replay_ms = e0.elapsed_time(e1)
    # per-kernel durations: the same steps launched eagerly on the same stream, HIP events between the kernels
    flush()
    torch.cuda.synchronize()
    for s in range(steps):
        stack.call(s % L, xs[s % L], ys[s % L], T, traces[s])
    torch.cuda.synchronize()
    stage_ms = [[he.elapsed_ms(events[s][i], events[s][i + 1]) for i in range(S.STAGE_EVENTS - 1)]
                for s in range(steps)]
    step_ms = [he.elapsed_ms(events[s][0], events[s][-1]) for s in range(steps)]
    D = (counts > 0).sum(dim=1).cpu().tolist()
    return dict(wall=wall, replay_ms=replay_ms, stage_ms=stage_ms, step_ms=step_ms, touched=D)


def bytes_model(S, g, T, D):
    """Algorithmic (compulsory) HBM bytes of one layer call touching D distinct experts, and of its gate/up and
    down kernels: weights of the touched experts and the shared expert, the router, x and y, and the activation
    images the kernels exchange (q8_1 images of x and h; the down kernel's f32 rows when they go through HBM)."""
    rb_h = S.row_bytes(g.w_type, g.n_embd)
    rb_f = S.row_bytes(g.w_type, g.n_ff)
    sh = g.sh_type >= 0
    Fs = g.n_ff_shared
    xq = T * g.n_embd // 32 * 36
    P = T * g.top_k
    hq = (P + (T if sh else 0)) * (max(g.n_ff, Fs if sh else 0) // 32) * 36
    gu = D * 2 * g.n_ff * rb_h + (2 * Fs * S.row_bytes(g.sh_type, g.n_embd) if sh else 0) + xq + hq
    down = D * g.n_embd * rb_f + (g.n_embd * S.row_bytes(g.sh_type, Fs) if sh else 0) + hq + (P + T) * g.n_embd * 4
    router_b = g.n_expert * g.n_embd * (4 if g.router_dtype == 1 else 2)
    layer = (D * g.expert_bytes() + g.shared_bytes() + router_b + (g.n_embd * 2 if sh else 0) + 2 * T * g.n_embd * 4)
    return layer, gu, down


def prefill_flops(g, T):
    """Dense FLOPs of one prefill call (2 * MACs): every routed pair and shared token through gate, up and down;
    the gate/up part alone; and the router."""
    P = T * g.top_k
    sh = g.sh_type >= 0
    gu = 2 * P * 2 * g.n_embd * g.n_ff + (2 * T * 2 * g.n_embd * g.n_ff_shared if sh else 0)
    down = 2 * P * g.n_embd * g.n_ff + (2 * T * g.n_embd * g.n_ff_shared if sh else 0)
    return gu + down, gu, 2 * T * g.n_embd * (g.n_expert + (1 if sh else 0))


def fused_small(g, T):
    """Batches of at most 4 Q2_0 tokens run as the router plus one launch (k_q2_moe_small: routing, gate/up, down and
    the combine) at the benchmark geometry."""
    return T <= 4 and g.w_type == 42


def fused_bytes(g, T, D):
    """Algorithmic HBM bytes of k_q2_moe_small: the gate, up and down rows of the D touched experts and of the shared
    expert, the q8_1 images of x and the logits it reads, and y (the h images stay on chip: LDS and the exchange)."""
    return (D * g.expert_bytes() + g.shared_bytes() + T * g.n_embd // 32 * 48 + T * g.n_expert * 4
            + T * g.n_embd * 4)


def summarize(S, g, T, r, steps):
    import statistics as st
    per_stage = {name: st.fmean(r["stage_ms"][s][i] for s in range(steps)) for i, name in enumerate(S.STAGES)}
    D = st.fmean(r["touched"])
    layer_b, gu_b, down_b = bytes_model(S, g, T, D)
    if fused_small(g, T):  # the gate_up stage is the one fused launch; the down and combine stages are empty
        gu_b, down_b = fused_bytes(g, T, D), 0
    ms = r["wall"] * 1e3 / steps
    gu_ms, down_ms = per_stage["gate_up"], per_stage["down"]
    return dict(tokens=T, ms_per_step=ms, tok_s=T * steps / r["wall"], gpu_ms_per_step=r["replay_ms"] / steps,
                touched_experts_avg=D, layer_bytes_avg=layer_b, layer_gbs=layer_b / (ms * 1e-3) / 1e9,
                layer_hbm_frac=layer_b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                stage_ms_avg=per_stage, gate_up_bytes=gu_b, down_bytes=down_b,
                gate_up_gbs=gu_b / (gu_ms * 1e-3) / 1e9 if gu_ms > 0 else None,
                down_gbs=down_b / (down_ms * 1e-3) / 1e9 if down_ms > 0 and down_b else None,
                step_event_ms_avg=st.fmean(r["step_ms"]))


def stage_line(name, m):
    return "%s: %.4f ms/step (GPU %.4f), %.0f tok/s, layer %.0f GB/s, touched %.1f, stages(us) %s" % (
        name, m["ms_per_step"], m["gpu_ms_per_step"], m["tok_s"], m["layer_gbs"], m["touched_experts_avg"],
        {k: round(v * 1e3, 2) for k, v in m["stage_ms_avg"].items()})


def decode(S, torch, stack, T, a, flush, seed_off):
    r = measure(S, torch, stack, T, a.steps, a.warmup, a.seed + seed_off, flush)
    m = summarize(S, stack.g, T, r, a.steps)
    log(stage_line(f"decode b={T}" + (" (f32 router)" if stack.g.router_dtype == 1 else ""), m))
    return m


def prefill(S, torch, g, a, flush):
    """512 tokens per call, expert popularity Zipf(1.2) through a fitted router logit bias, the MFMA
    (prefill) contract.  `--prefill-layers` biased layers are resident; steps walk through them."""
    T = 512
    bias = S.zipf_bias(g.n_expert, 1.2, a.seed, n_tokens=T, top_k=g.top_k, n_embd=g.n_embd)
    t0 = time.perf_counter()
    stack = Stack(S, torch, g, a.prefill_layers, a.seed + 1000, T, logit_bias=torch.from_numpy(bias).cuda())
    log(f"prefill: {a.prefill_layers} Zipf-biased layers resident in {time.perf_counter() - t0:.1f} s")
    steps = a.prefill_steps
    r = measure(S, torch, stack, T, steps, max(2, steps // 3), a.seed + 13, flush)
    m = summarize(S, g, T, r, steps)
    ex_flops, gu_flops, router_flops = prefill_flops(g, T)
    st = m["stage_ms_avg"]
    mm_ms = st["gate_up"] + st["down"]
    out = {k: m[k] for k in ("ms_per_step", "gpu_ms_per_step", "tok_s", "touched_experts_avg", "layer_bytes_avg",
                             "layer_gbs", "layer_hbm_frac", "stage_ms_avg")}
    out["expert_flops"] = ex_flops
    out["router_flops"] = router_flops
    out["expert_gemm_tflops"] = ex_flops / (mm_ms * 1e-3) / 1e12
    out["expert_gemm_mfma_frac"] = out["expert_gemm_tflops"] / BF16_PEAK_TFLOPS
    out["layer_tflops"] = (ex_flops + router_flops) / (m["ms_per_step"] * 1e-3) / 1e12
    gu_tf = gu_flops / (st["gate_up"] * 1e-3) / 1e12
    # the binding roof of k_mm_gu: its compulsory bytes (the touched experts' and the shared expert's gate and up
    # rows, x as fp16 records, h records written) at 8 TB/s against its useful FLOPs at 2.5 PFLOP/s; with Zipf(1.2)
    # routing most touched experts get a few tokens, and the weight bytes take longer than the matrix work
    D = m["touched_experts_avg"]
    P = T * g.top_k
    rb_h = S.row_bytes(g.w_type, g.n_embd)
    gu_bytes = (D * 2 * g.n_ff * rb_h + 2 * g.n_ff_shared * S.row_bytes(g.sh_type, g.n_embd) + T * g.n_embd * 2
                + (P + T) * max(g.n_ff, g.n_ff_shared) * 2)
    t_hbm_us = gu_bytes / (HBM_PEAK_GBS * 1e9) * 1e6
    t_mfma_us = gu_flops / (BF16_PEAK_TFLOPS * 1e12) * 1e6
    gu_gbs = gu_bytes / (st["gate_up"] * 1e-3) / 1e9
    common = {"kernel": "k_mm_gu + k_mm_gu_thin (the gate/up stage: routed + shared gate/up, SwiGLU, bf16 h "
                        "records; the items of at most 16 columns in a kernel of their own)", "traffic": None,
              "algorithmic_bytes_per_launch": gu_bytes, "useful_flops_per_launch": gu_flops,
              "avg_launch_ms": st["gate_up"], "roof_us": {"hbm": t_hbm_us, "mfma": t_mfma_us},
              "mfma_tflops": gu_tf, "mfma_frac": gu_tf / BF16_PEAK_TFLOPS, "hbm_gbs": gu_gbs,
              "hbm_frac": gu_gbs / HBM_PEAK_GBS, "mfma_busy": None}
    if t_hbm_us >= t_mfma_us:
        roof = dict({"bound": "hbm", "achieved": gu_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gu_gbs / HBM_PEAK_GBS}, **common)
    else:
        roof = dict({"bound": "mfma", "achieved": gu_tf, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": gu_tf / BF16_PEAK_TFLOPS}, **common)
    rec = profile_record("prefill512_counters", "smoe::k_mm_gu")
    if rec:
        roof["traffic"] = rec.get("traffic_bytes")
        roof["mfma_busy"] = rec.get("mfma_busy")
        roof["counters_source"] = "profiles/prefill512_counters.md"
    out["roofline"] = roof
    log(stage_line("prefill 512", m) + ", expert GEMMs %.0f TFLOP/s (%.1f%% of bf16 peak), k_mm_gu %.0f TFLOP/s, "
        "%.0f GB/s (%s-bound: roofs %.1f us HBM, %.1f us MFMA)"
        % (out["expert_gemm_tflops"], 100 * out["expert_gemm_mfma_frac"], gu_tf, gu_gbs, roof["bound"], t_hbm_us,
           t_mfma_us))
    del stack
    torch.cuda.empty_cache()
    return out


def stack48(S, torch, g, stack, a):
    """the resident layers chained as x_{l+1} = RMSNorm(x_l + MoE_l(x_l)) (unit weight, eps 1e-6):
    one `--stack-prefill` token prefill through every layer (the MFMA contract), then `--stack-decode` decode
    steps at batch 1 (each step one graph of every layer and junction, replayed on a fresh token).  Each
    junction after the first layer runs inside the next layer's call (smoe_forward_residual, bitwise equal to
    the separate junction and call), the last one on its own."""
    import ctypes as C
    L = len(stack.layers)
    H, Tp, steps = g.n_embd, a.stack_prefill, a.stack_decode
    ws_bytes = S.workspace_bytes(g, Tp)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    lib = S.lib()

    def chain(xa, xb, y, T):
        """Every layer on xa (xb the other junction buffer, y the layer output); the final x ends in xa or xb."""
        S._check(lib.smoe_forward(C.byref(stack.gc), C.byref(stack.wc[0]), xa.data_ptr(), T, y.data_ptr(), 1,
                                  ws.data_ptr(), ws_bytes, None, S._stream()))
        cur, nxt = xa, xb
        for l in range(1, L):
            S._check(lib.smoe_forward_residual(C.byref(stack.gc), C.byref(stack.wc[l]), cur.data_ptr(),
                                               y.data_ptr(), C.c_float(1e-6), nxt.data_ptr(), T, y.data_ptr(), 1,
                                               ws.data_ptr(), ws_bytes, None, S._stream()))
            cur, nxt = nxt, cur
        S.residual_rmsnorm(cur, y, 1e-6, out=cur)
        return cur

    x0 = S.synth_normal(a.seed + 40, 100, Tp * H).view(Tp, H)
    x = torch.empty_like(x0)
    x2 = torch.empty_like(x0)
    y = torch.empty_like(x0)
    times = []
    for rep in range(2):  # the first pass loads code and warms the allocator; the second is the measurement
        x.copy_(x0)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        ev0.record()
        xl = chain(x, x2, y, Tp)
        ev1.record()
        torch.cuda.synchronize()
        times.append(ev0.elapsed_time(ev1))
    pre_ms = times[-1]
    ex_flops, _, router_flops = prefill_flops(g, Tp)
    out = {"layers": L, "prefill_tokens": Tp, "prefill_ms": pre_ms, "prefill_tok_s": Tp / (pre_ms * 1e-3),
           "prefill_tflops": L * (ex_flops + router_flops) / (pre_ms * 1e-3) / 1e12,
           "prefill_out_finite": bool(torch.isfinite(xl).all().item())}
    # decode: one graph per step over every layer, replayed on fresh tokens
    xs = S.synth_normal(a.seed + 41, 100, steps * H).view(steps, H)
    xin = torch.empty((1, H), dtype=torch.float32, device="cuda")
    xalt = torch.empty((1, H), dtype=torch.float32, device="cuda")
    yb = torch.empty((1, H), dtype=torch.float32, device="cuda")
    xin.copy_(xs[0:1])
    chain(xin, xalt, yb, 1)  # eager pass (code and workspace warm)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    gs = torch.cuda.Stream()
    gs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(gs):
        with torch.cuda.graph(graph, stream=gs):
            chain(xin, xalt, yb, 1)
    torch.cuda.synchronize()
    xin.copy_(xs[0:1])
    graph.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for s in range(steps):
        xin.copy_(xs[s:s + 1])
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    dec_ms = ev0.elapsed_time(ev1)
    per_tok = dec_ms / steps
    tok_bytes = L * bytes_model(S, g, 1, g.top_k)[0]
    out.update({"decode_steps": steps, "decode_ms_per_token": per_tok, "decode_tok_s": 1e3 / per_tok,
                "decode_bytes_per_token": tok_bytes, "decode_gbs": tok_bytes / (per_tok * 1e-3) / 1e9})
    out["decode_hbm_frac"] = out["decode_gbs"] / HBM_PEAK_GBS
    log("stack of %d: prefill %d tokens %.2f ms (%.0f tok/s, %.0f TFLOP/s), decode %.3f ms/token (%.0f tok/s, "
        "%.0f GB/s)" % (L, Tp, pre_ms, out["prefill_tok_s"], out["prefill_tflops"], per_tok, out["decode_tok_s"],
                        out["decode_gbs"]))
    del ws, x, x2, y, x0
    torch.cuda.empty_cache()
    return out


def iq2_b64(S, torch, a, flush):
    """batch 64, IQ2_S routed and shared experts, uniform routing (no bias), decode contract.
    `--iq2-layers` resident layers (about 0.5 GB each) so that steps do not hit the Infinity Cache."""
    g = S.Geom(w_type=S.IQ2_S, sh_type=S.IQ2_S)
    t0 = time.perf_counter()
    stack = Stack(S, torch, g, a.iq2_layers, a.seed + 2000, 64)
    log(f"IQ2_S: {a.iq2_layers} layers resident in {time.perf_counter() - t0:.1f} s")
    steps = a.prefill_steps
    r = measure(S, torch, stack, 64, steps, max(2, steps // 3), a.seed + 17, flush)
    m = summarize(S, g, 64, r, steps)
    out = {k: m[k] for k in ("ms_per_step", "gpu_ms_per_step", "tok_s", "touched_experts_avg", "layer_bytes_avg",
                             "layer_gbs", "layer_hbm_frac", "stage_ms_avg", "gate_up_gbs", "down_gbs")}
    log(stage_line("IQ2_S b=64", m))
    del stack
    torch.cuda.empty_cache()
    return out


def cpu_baseline(S, a):
    """The reference CPU path, restated: the test oracle's decode contract organised as the reference's CPU pool
    (flat (expert, row-range) jobs per stage, one worker per core, each weight row decoded once for all of its
    expert's tokens; oracle/smoe_cpu_pool.c), compiled with -O3 -march=native for this host and timed on it, with
    every core of this GPU's share and with 1 thread, on configs[0] (b=1), configs[1] (b=16) and configs[3]
    (IQ2_S b=64), each on one synthetic layer with a fresh batch per call; and configs[2] (prefill 512) through the
    oracle's prefill contract."""
    import oracle as O
    cores = max(1, min(16, len(os.sched_getaffinity(0))))
    tmp = tempfile.mkdtemp(prefix="smoe_cpu_")
    lib_path = os.path.join(tmp, "liboracle_native.so")
    built = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "native", f"OUT={lib_path}"],
                           capture_output=True, text=True)
    if built.returncode == 0:
        lib, flags = O.load_library(lib_path), "-O3 -march=native"
    else:
        lib, flags = O.lib(), "-O3 -march=x86-64-v3 (the native build failed)"
    try:
        model = [l for l in open("/proc/cpuinfo") if l.startswith("model name")][0].split(":", 1)[1].strip()
    except (OSError, IndexError):
        model = "unknown"
    out = {"cores": cores, "nproc": os.cpu_count(), "cpu_model": model, "build": flags}
    work = [("b1", O.Geom(), 1), ("b16", O.Geom(), 16), ("iq2_s_b64", O.Geom(w_type=O.IQ2_S, sh_type=O.IQ2_S), 64)]
    for name, og, T in work:
        w = O.make_weights(og, a.seed + 3000)
        sg = S.Geom(**{k: getattr(og, k) for k in ("n_embd", "n_ff", "n_ff_shared", "n_expert", "top_k", "w_type",
                                                   "sh_type")})
        for threads in (cores, 1):
            n, el, D_sum = 0, 0.0, 0.0
            while el < a.cpu_seconds and n < 400:
                x = O.gen_normal(a.seed + 3001, 1000 + n, T * og.n_embd).reshape(T, og.n_embd)
                t0 = time.perf_counter()
                O.moe_decode_pool(og, w, x, n_threads=threads, library=lib)
                el += time.perf_counter() - t0
                n += 1
            # bytes: the expected distinct experts of uniform top-k routing (the seeded router is close to it)
            E, K = og.n_expert, og.top_k
            D = E * (1 - (1 - K / E) ** T)
            tok_s = T * n / el
            gbs = bytes_model(S, sg, T, D)[0] * n / el / 1e9
            out[f"{name}_threads{threads}"] = {"tok_s": tok_s, "layer_gbs": gbs, "calls": n, "seconds": el}
            log(f"cpu baseline {name}, {threads} threads: {tok_s:.1f} tok/s, {gbs:.2f} GB/s ({n} calls)")
    # configs[2] (prefill 512, Zipf(1.2) routing as in the GPU leg): the oracle's prefill contract (or_moe_prefill,
    # OpenMP over tokens, each token's experts in turn), the whole batch with every core and a 64-token sample of
    # the same batch with one thread
    og = O.Geom()
    bias = S.zipf_bias(og.n_expert, 1.2, a.seed, n_tokens=512, top_k=og.top_k, n_embd=og.n_embd)
    w = O.make_weights(og, a.seed + 3000, zipf_bias=bias)
    x = O.gen_normal(a.seed + 3002, 1, 512 * og.n_embd).reshape(512, og.n_embd)
    for threads, T in ((cores, 512), (1, 64)):
        t0 = time.perf_counter()
        O.moe_prefill(og, w, x[:T], n_threads=threads)
        el = time.perf_counter() - t0
        out[f"prefill512_threads{threads}"] = {"tok_s": T / el, "tokens": T, "seconds": el,
                                               "path": "oracle or_moe_prefill (liboracle.so)"}
        log(f"cpu baseline prefill512, {threads} threads: {T / el:.1f} tok/s ({T} tokens)")
    head = out[f"b1_threads{cores}"]
    return {"value": head["tok_s"], "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": (f"configs[0] (decode b=1): {head['calls']} layer calls on one synthetic layer, each on a fresh "
                       f"token ({head['seconds']:.1f} s), oracle/smoe_cpu_pool.c (the reference host path as the "
                       f"reference CPU pool runs it), {flags}, {cores} OpenMP threads on {model}"),
            "detail": out}


def main():
    a = _args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {a.gpus} is not supported (the path is "
              f"single-GPU by design; across GPUs it would shard by expert, with an all-to-all of the "
              f"dispatched rows each way)", file=sys.stderr)
        sys.exit(2)
    import ctypes
    import torch
    if a.copy_calibration:
        n = a.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {a.copy_calibration} MiB x5")
        return
    import stratametal_amd as S
    S.C = ctypes
    g = S.Geom()
    flush = Flush(torch, a.flush)
    if a.only == "prefill":
        prefill(S, torch, g, a, flush)
        return
    if a.only == "iq2":
        iq2_b64(S, torch, a, flush)
        return
    t_setup = time.perf_counter()
    stack = Stack(S, torch, g, a.layers, a.seed, 16)
    log(f"{a.layers} layers resident ({a.layers * (g.n_expert * g.expert_bytes() + g.shared_bytes()) / 1e9:.1f} GB) "
        f"in {time.perf_counter() - t_setup:.1f} s")
    if a.only == "stack":
        stack48(S, torch, g, stack, a)
        return
    if a.only == "b16":
        decode(S, torch, stack, 16, a, flush, 7)
        return
    m1 = decode(S, torch, stack, 1, a, flush, 11)
    if a.only == "b1":
        return
    extra = {}
    if not a.no_extra:
        # the literal configs[0]: the same layers and tokens with the f32 router (4 MiB of router rows per layer)
        st32 = stack.with_f32_router()
        m1f = decode(S, torch, st32, 1, a, flush, 11)
        extra["decode_b1_f32_router"] = {k: m1f[k] for k in ("ms_per_step", "gpu_ms_per_step", "tok_s",
                                                             "touched_experts_avg", "layer_bytes_avg", "layer_gbs",
                                                             "layer_hbm_frac", "stage_ms_avg")}
        del st32
        m16 = decode(S, torch, stack, 16, a, flush, 7)
        extra["decode_b16"] = {k: m16[k] for k in ("ms_per_step", "gpu_ms_per_step", "tok_s", "touched_experts_avg",
                                                   "layer_bytes_avg", "layer_gbs", "layer_hbm_frac", "stage_ms_avg",
                                                   "gate_up_gbs", "down_gbs")}
        extra["stack48"] = stack48(S, torch, g, stack, a)
        del stack
        torch.cuda.empty_cache()
        extra["prefill_512"] = prefill(S, torch, g, a, flush)
        extra["iq2_s_b64"] = iq2_b64(S, torch, a, flush)
    extra["decode_b1"] = {k: m1[k] for k in ("gpu_ms_per_step", "touched_experts_avg", "layer_bytes_avg", "layer_gbs",
                                             "layer_hbm_frac", "stage_ms_avg", "step_event_ms_avg", "gate_up_gbs",
                                             "down_gbs")}
    gu_ms = m1["stage_ms_avg"]["gate_up"]
    roof = {"bound": "hbm",
            "kernel": "k_q2_moe_small (routes the token; routed + shared gate/up, SwiGLU, q8_1 of h; down rows and the "
                      "combine)",
            "achieved": m1["gate_up_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": m1["gate_up_gbs"] / HBM_PEAK_GBS, "traffic": None,
            "algorithmic_bytes_per_launch": m1["gate_up_bytes"], "avg_launch_ms": gu_ms}
    rec = profile_record("decode_b1_traffic", "smoe::k_q2_moe_small")
    if rec:  # HBM bytes per launch from the FETCH_SIZE / WRITE_SIZE counter runs (calibrated), same sources only
        roof["traffic"] = rec["traffic_bytes"]
        roof["traffic_source"] = "profiles/decode_b1_traffic.md"
    cpu = None if a.no_cpu else cpu_baseline(S, a)
    out = {
        "metric": METRIC, "value": m1["tok_s"], "unit": "tokens/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": m1["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 (q8_1 x Q2_0 integer dot, f32 scale and sums)", "data": "synthetic",
        "config": {"workload": "BASELINE configs[0]: one Qwen3-Next-style MoE layer decoding 1 token",
                   "tokens_per_step": 1, "n_embd": g.n_embd, "n_ff": g.n_ff, "n_expert": g.n_expert,
                   "top_k": g.top_k, "shared_experts": 1, "expert_type": "Q2_0", "router": "bf16",
                   "resident_layers": a.layers, "cache": f"1 GiB {'read' if a.flush == 'read' else 'rewritten'} before the timed replay",
                   "parallelism": "none (1 GPU)"},
        "roofline": roof, "roofline_prefill_512": extra.get("prefill_512", {}).get("roofline"),
        "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
