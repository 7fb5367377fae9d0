"""Writes the committed golden fixtures under tests/golden/.

    python tests/golden/gen_golden.py

codecs_ref.npz       f16 / bf16 encodings of edge-case floats and Q2_0 dequantisations computed by the
                     REFERENCE's own header-only code (oracle/_ref/libsmoe_ref.so, compiled from
                     include/strata/kernels/{f16,bf16}_bits.hpp and include/strata/artifact/dequant.hpp),
                     so the codec checks hold on machines without /root/reference.
layer_small.npz      one small seeded layer through the oracle's device-order decode contract: input, output,
                     routing trace and sha256 of every generated tensor (pins the generators and the chain).
layer_prefill.npz    the same layer through the prefill contract (bf16 activations, exact block scales).
native_ref.npz       blocks of the other native GGUF types (Q8_0, Q4_0, Q5_0, IQ4_NL, IQ4_XS, Q3_K, Q4_K, Q5_K, Q6_K)
                     and their values as the REFERENCE's own dequantisers give them (include/strata/artifact/
                     dequant.hpp:81-280 through oracle/_ref), edge scales included.

    python tests/golden/gen_golden.py native     # writes native_ref.npz alone
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402


def edge_floats():
    v = [0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 65519.99, 65536.0, 1e30, -1e30, 6.1035156e-05, 6.0975552e-05,
         5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-8, 1e-45, 0.1, 1.0 / 3.0, 3.14159265, 1e-3, 2048.5, 2049.0,
         float("inf"), float("-inf"), float("nan")]
    # exact fp16 / bf16 ties and their neighbours
    for base in (1.0, 1024.0, 3.0e-5, 0.5, 7.0):
        u = np.array([base], np.float32).view(np.uint32)[0]
        for d in (0x0FFF, 0x1000, 0x1001, 0x2000 + 0x1000, 0x7FFF, 0x8000, 0x8001, 0x18000):
            v.append(float(np.array([u + d], np.uint32).view(np.float32)[0]))
    rng = np.random.default_rng(20261014)
    r = rng.integers(0, 2 ** 32, 4000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return np.concatenate([np.array(v, np.float32), r])


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    O.build()
    R = O.ref()
    if R is None:
        raise SystemExit("oracle/_ref is not built (needs /root/reference): cannot write the reference codec vectors")
    x = edge_floats()
    f16 = np.empty(x.size, np.uint16)
    bf16 = np.empty(x.size, np.uint16)
    R.ref_f16_from_f32_n(x.ctypes.data, x.size, f16.ctypes.data)
    R.ref_bf16_from_f32_n(x.ctypes.data, x.size, bf16.ctypes.data)
    f16_all = np.empty(65536, np.float32)
    R.ref_f32_from_f16_all(f16_all.ctypes.data)
    blocks = O.gen_q2_0(99, 7, 64)
    blocks[0:2] = [0x01, 0x00]      # smallest subnormal scale
    blocks[18:20] = [0x00, 0x80]    # -0 scale
    blocks[36:38] = [0xFF, 0x7B]    # 65504
    deq = np.empty(64 * 64, np.float32)
    R.ref_dequantize_q2_0(blocks.ctypes.data, 64, deq.ctypes.data)
    grid = np.empty(1024, np.uint64)
    R.ref_iq2s_grid(grid.ctypes.data)
    np.savez_compressed(os.path.join(HERE, "codecs_ref.npz"), x=x, f16=f16, bf16=bf16,
                        f16_decode_sha=np.array(sha(f16_all)), q2_blocks=blocks, q2_dequant=deq,
                        iq2s_grid_sha=np.array(sha(grid)))

    g = O.Geom(n_embd=256, n_ff=128, n_ff_shared=128, n_expert=16, top_k=4)
    seed = 4242
    w = O.make_weights(g, seed)
    xin = O.gen_normal(seed, 100, 3 * g.n_embd).reshape(3, g.n_embd)
    y, tr = O.moe_decode_dev(g, w, xin, trace=True)
    yp, trp = O.moe_prefill(g, w, xin, trace=True)
    hashes = {n: sha(getattr(w, n)) for n in ("gate_exps", "up_exps", "down_exps", "router", "gate_sh", "up_sh",
                                              "down_sh", "gate_inp_sh")}
    geom = np.array([g.n_embd, g.n_ff, g.n_ff_shared, g.n_expert, g.top_k, g.w_type, g.sh_type, seed], np.int64)
    np.savez_compressed(os.path.join(HERE, "layer_small.npz"), geom=geom, x=xin, y=y,
                        **{k: tr[k] for k in ("logits", "ids", "weights", "counts", "offsets", "perm", "slot",
                                              "sgate", "xq")},
                        **{"sha_" + k: np.array(v) for k, v in hashes.items()})
    np.savez_compressed(os.path.join(HERE, "layer_prefill.npz"), geom=geom, x=xin, y=yp,
                        **{k: trp[k] for k in ("logits", "ids", "weights")})
    for f in ("codecs_ref.npz", "layer_small.npz", "layer_prefill.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


def native_blocks(t: int) -> np.ndarray:
    """Seeded blocks of type t plus edge scale fields: the smallest subnormal, -0, 65504, and a zero block."""
    qk, nb, fields, _ = O.NATIVE[t]
    b = O.gen_native_blocks(t, 20261202, 77, 12 * qk).reshape(12, nb).copy()
    for f in fields:
        b[0, f:f + 2] = [0x01, 0x00]
        b[1, f:f + 2] = [0x00, 0x80]
        b[2, f:f + 2] = [0xFF, 0x7B]
    b[3] = 0
    return b.ravel()


def main_native():
    O.build()
    if O.ref() is None:
        raise SystemExit("oracle/_ref is not built (needs /root/reference): cannot write the reference vectors")
    out = {}
    for t in sorted(O.NATIVE):
        b = native_blocks(t)
        n = b.size // O.NATIVE[t][1] * O.NATIVE[t][0]
        out[f"blocks_{t}"] = b
        out[f"values_{t}"] = O.ref_dequantize(t, b, n)
    np.savez_compressed(os.path.join(HERE, "native_ref.npz"), **out)
    print("native_ref.npz", os.path.getsize(os.path.join(HERE, "native_ref.npz")), "bytes")


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "native":
        main_native()
    else:
        main()
