"""The decode layer's phase timeline: when each work-group of the router and of the fused decode launch reaches each
phase, from the 100 MHz clock every work-group reads (s_memrealtime), on a build of the library with its phase
stamps compiled in (SMOE_STAMPS; lib/libsmoe_stamps.so, never the product library).

    python -m stratametal_amd.timeline build            # here: lib/libsmoe_stamps.so from the built objects
    python -m stratametal_amd.timeline run [--tokens 1]  # on the GPU: the table, in microseconds

The layer is configs[0]'s geometry (hidden 2048, 512 experts + the shared one, top-10, n_ff 512, Q2_0), twelve
distinct synthetic layers taken in turn so that the weights come from HBM, and the memory-side cache flushed
(a 1 GiB read) before each call; with `--no-flush --layers 48` the calls follow each other as in the benchmark's
replay (the code and the workspace stay cached, the weights of 48 layers do not).  Per phase: the median and the maximum over the role's work-groups, each the
median over the measured calls; times from the first router work-group's start.  A stamp costs its work-group
a clock read and a store (~0.1-0.3 us), so the phases run later than in the product build by up to that much per
stamp passed.
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys

from . import build as B

LIB_STAMPS = os.path.join(B.LIBDIR, "libsmoe_stamps.so")
ROLES = {0: "router", 1: "gate/up (shared)", 2: "gate/up (routed)", 9: "gate/up (no expert)", 3: "writer",
         4: "down"}
PHASES = [(2, "start"), (3, "dots begin"), (15, "image loads issued"), (4, "sg loaded"), (13, "logits in registers"),
          (14, "routed"),
          (6, "item known"), (7, "weights in registers"), (8, "h words polled"), (9, "h seen"),
          (11, "first rows formed"), (12, "rows parked"), (10, "end")]


def build(verbose: bool = True) -> str:
    """lib/libsmoe_stamps.so: smoe_decode.hip with SMOE_STAMPS, linked with the other objects of the build."""
    out_dir = os.path.join(B.BUILD, "stamps")
    os.makedirs(out_dir, exist_ok=True)
    obj = os.path.join(out_dir, "smoe_decode.o")
    cmd = [B.HIPCC, *B.COMMON, "-DSMOE_STAMPS", "-c", os.path.join(B.CSRC, "smoe_decode.hip"), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr[-4000:])
    rest = [os.path.join(B.BUILD, os.path.splitext(s)[0] + ".o") for s in B.SOURCES if s != "smoe_decode.hip"]
    missing = [o for o in rest if not os.path.exists(o)]
    if missing:
        raise RuntimeError(f"build the library first (python -m stratametal_amd.build): {missing[0]} is missing")
    tmp = LIB_STAMPS + ".tmp"
    r = subprocess.run([B.HIPCC, f"--offload-arch={B.ARCH}", "-shared", "-fPIC", "-o", tmp, obj, *rest],
                       capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr[-4000:])
    os.replace(tmp, LIB_STAMPS)
    if verbose:
        print("built", LIB_STAMPS)
    return LIB_STAMPS


def run(tokens: int = 1, reps: int = 12, warm: int = 4, n_layers: int = 12, flush_each: bool = True) -> str:
    import ctypes as C

    import numpy as np

    import stratametal_amd as S
    if not os.path.exists(LIB_STAMPS):
        raise ImportError(f"{LIB_STAMPS} is missing: python -m stratametal_amd.timeline build")
    S.LIB_PATH = LIB_STAMPS
    S._LIB = None
    import torch
    L = S.lib()
    L.smoe_debug_set_stamps.argtypes = [C.c_void_p]
    L.smoe_debug_set_stamps.restype = C.c_int
    g = S.Geom()
    layers = [S.synth_layer(g, 1000 + i) for i in range(n_layers)]
    ml = S.MoELayer(g, layers[0], max_tokens=tokens)
    flush = torch.zeros((1 << 30) // 4, dtype=torch.float32, device="cuda")
    st = torch.zeros(2 * 4096 * 32, dtype=torch.int64, device="cuda")
    assert L.smoe_debug_set_stamps(st.data_ptr()) == 0
    xs = [torch.randn(tokens, g.n_embd, device="cuda") for _ in range(n_layers)]
    acc = {}
    ends = []
    try:
        for rep in range(reps + warm):
            ml._wc = S._weights_c(layers[rep % n_layers])
            if flush_each or rep == 0:
                sink = flush.sum()
            torch.cuda.synchronize()
            st.zero_()
            torch.cuda.synchronize()
            ml.forward(xs[rep % n_layers])
            torch.cuda.synchronize()
            a = st.cpu().numpy().reshape(2, 4096, 32)
            r, f = a[0], a[1]
            ur, uf = r[:, 2] > 0, f[:, 2] > 0
            t0 = r[ur, 2].min()
            if rep < warm:
                continue
            ends.append((f[uf, 10].max() - t0) / 100)
            groups = [(0, r[ur])] + [(role, f[uf & (f[:, 0] == role)]) for role in (1, 2, 9, 3, 4)]
            for role, blk in groups:
                if len(blk) == 0:
                    continue
                acc.setdefault((role, "n"), []).append(len(blk))
                for c, _ in PHASES:
                    v = blk[:, c]
                    v = v[v > 0]
                    if v.size:
                        acc.setdefault((role, c), []).append(((np.median(v) - t0) / 100, (v.max() - t0) / 100))
        del sink
    finally:
        L.smoe_debug_set_stamps(None)
    lines = [f"decode T={tokens}, configs[0] geometry, {n_layers} layers in turn, "
             f"{'memory-side cache flushed before each call' if flush_each else 'no flush between calls'}, {reps} calls "
             f"after {warm} warm-up calls; last work-group end {np.median(ends):.2f} us (median over calls, from the "
             f"first router work-group's start)", "",
             "| role | work-groups | phase | median us | max us |", "|---|---|---|---|---|"]
    for role, name in ROLES.items():
        if (role, "n") not in acc:
            continue
        n = int(np.median(acc[(role, "n")]))
        first = True
        for c, pname in PHASES:
            if (role, c) not in acc:
                continue
            v = np.array(acc[(role, c)])
            lines.append(f"| {name if first else ''} | {n if first else ''} | {pname} | "
                         f"{np.median(v[:, 0]):.2f} | {np.median(v[:, 1]):.2f} |")
            first = False
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("what", choices=("build", "run"))
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--reps", type=int, default=12)
    ap.add_argument("--layers", type=int, default=12, help="distinct synthetic layers taken in turn")
    ap.add_argument("--no-flush", action="store_true", help="no cache flush between calls (the bench's replay: "
                    "use enough layers that their weights exceed the Infinity Cache)")
    a = ap.parse_args(argv)
    if a.what == "build":
        build()
    else:
        print(run(a.tokens, a.reps, n_layers=a.layers, flush_each=not a.no_flush), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
