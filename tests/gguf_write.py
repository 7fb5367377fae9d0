"""A GGUF v3 writer for the tests: synthetic models (one file or split shards) with any metadata and tensors, and
deliberately malformed ones.  The layout is the GGUF v3 file format (header, metadata, tensor directory, the data
section at general.alignment); the reader under test is smoe_model_* (stratametal_amd/csrc/smoe_gguf.cpp)."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
        F64: "<d"}

# GGUF tensor types used here
T_F32, T_F16, T_BF16, T_Q2_0, T_IQ2_S = 0, 1, 30, 42, 22


def gstr(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(t: int, v) -> bytes:
    if t == STRING:
        return gstr(v)
    if t == ARRAY:
        elem, items = v
        return struct.pack("<IQ", elem, len(items)) + b"".join(value(elem, x) for x in items)
    return struct.pack(_FMT[t], v)


class Tensor:
    """One directory entry: `ne` in GGUF order (ne[0] varies fastest), the payload bytes, and optionally an
    explicit offset into the data section (otherwise the next aligned one; an explicit one does not lengthen the
    file, so it can point past its end)."""

    def __init__(self, name: str, ne, type_: int, data, offset=None):
        self.name, self.ne, self.type, self.offset = name, tuple(int(n) for n in ne), type_, offset
        self.data = np.ascontiguousarray(data).tobytes() if not isinstance(data, (bytes, bytearray)) else bytes(data)


def build(meta, tensors, alignment: int = 32, version: int = 3, magic: bytes = b"GGUF") -> bytes:
    """The bytes of a GGUF file.  `meta` is a list of (key, type, value); arrays are (elem type, items)."""
    kv = b"".join(gstr(k) + struct.pack("<I", t) + value(t, v) for k, t, v in meta)
    offs, at = [], 0
    for t in tensors:
        if t.offset is None:
            at = (at + alignment - 1) // alignment * alignment
            offs.append(at)
            at += len(t.data)
        else:
            offs.append(t.offset)
    dirs = b"".join(gstr(t.name) + struct.pack("<I", len(t.ne)) + b"".join(struct.pack("<Q", n) for n in t.ne) +
                    struct.pack("<IQ", t.type, o) for t, o in zip(tensors, offs))
    head = magic + struct.pack("<IQQ", version, len(tensors), len(meta)) + kv + dirs
    start = (len(head) + alignment - 1) // alignment * alignment
    # the file ends after the last tensor placed here; one given an explicit offset may point past it
    end = max([o + len(t.data) for t, o in zip(tensors, offs) if t.offset is None], default=0)
    body = bytearray(end)
    for t, o in zip(tensors, offs):
        if o + len(t.data) <= end:
            body[o:o + len(t.data)] = t.data
    return head + b"\0" * (start - len(head)) + bytes(body)


def write(path, meta, tensors, **kw) -> str:
    with open(path, "wb") as f:
        f.write(build(meta, tensors, **kw))
    return str(path)


def split_name(stem, i: int, n: int) -> str:
    return f"{stem}-{i:05d}-of-{n:05d}.gguf"


def write_split(stem, meta, shards, arch: str = "test", keys=None):
    """A split model: shard 1 carries `meta` and general.architecture; every shard declares split.count,
    split.no and split.tensors.count (each overridable per shard through `keys[i]`).  Returns the paths."""
    n = len(shards)
    total = sum(len(s) for s in shards)
    paths = []
    for i, ts in enumerate(shards):
        k = {"split.count": (U16, n), "split.no": (U16, i), "split.tensors.count": (I32, total)}
        if keys and i in keys:
            k.update(keys[i])
        m = [(key, t, v) for key, (t, v) in k.items() if t is not None]
        if i == 0:
            m = [("general.architecture", STRING, arch)] + list(meta) + m
        p = split_name(stem, i + 1, n)
        write(p, m, ts)
        paths.append(p)
    return paths


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (NaN quieted)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = ((u[nan] >> 16) | 64).astype(np.uint16)
    return r


def layer_tensors(g, w, layer: int, router=None, gate_inp_sh=None, hc=None):
    """The MoE tensors of layer `layer` (blk.<L>.*) from the oracle's host weights `w` of geometry `g`:
    the routed planes [n_embd][n_ff][n_expert] (down [n_ff][n_embd][n_expert]), the router [n_embd][n_expert]
    (BF16, or F32 when router_dtype is 1), the shared planes and gate, and `hc` = (hc, hc_lr, norm f32, down,
    up, inject bf16 bits) when given.  `router` / `gate_inp_sh` replace the stored arrays (with their type)."""
    H, F, Fs, E = g.n_embd, g.n_ff, g.n_ff_shared, g.n_expert
    b = f"blk.{layer}."
    rt = T_F32 if g.router_dtype == 1 else T_BF16
    out = [Tensor(b + "ffn_gate_exps.weight", (H, F, E), g.w_type, w.gate_exps),
           Tensor(b + "ffn_up_exps.weight", (H, F, E), g.w_type, w.up_exps),
           Tensor(b + "ffn_down_exps.weight", (F, H, E), g.w_type, w.down_exps),
           Tensor(b + "ffn_gate_inp.weight", (H, E), rt, w.router) if router is None else
           Tensor(b + "ffn_gate_inp.weight", (H, E), router[0], router[1])]
    if g.sh_type >= 0:
        tg, tu, td = g.shared_types()
        out += [Tensor(b + "ffn_gate_shexp.weight", (H, Fs), tg, w.gate_sh),
                Tensor(b + "ffn_up_shexp.weight", (H, Fs), tu, w.up_sh),
                Tensor(b + "ffn_down_shexp.weight", (Fs, H), td, w.down_sh)]
        gi = (T_BF16, w.gate_inp_sh) if gate_inp_sh is None else gate_inp_sh
        out.append(Tensor(b + "ffn_gate_inp_shexp.weight", (H,), gi[0], gi[1]))
    if hc is not None:
        n, lr, norm, down, up, inject = hc
        out += [Tensor(b + "hc_ffn_norm.weight", (n * H,), T_F32, norm),
                Tensor(b + "hc_ffn_down.weight", (n * H, lr), T_BF16, down),
                Tensor(b + "hc_ffn_up.weight", (lr, n * H), T_BF16, up),
                Tensor(b + "hc_ffn_inject.weight", (n * H, n), T_BF16, inject)]
    return out
