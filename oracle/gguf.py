"""CPU restatement of the reference's GGUF reader and MoE tensor addressing.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the library's C++ reader
(garuda_amd/csrc/gmoe_gguf.cpp). The product never loads it.

Follows, in plain Python:
  * Gguf::parse and its Cursor, garuda/src/gguf/mod.rs:113-245 (reads, string and
    array bounds, min_value_bytes, nesting depth) and :247-324 (magic, version 2..=3,
    header count bounds of 24 and 13 bytes, metadata into an ordered map where a
    repeated key keeps the last value, tensor descriptors with at most 4 dims, data
    offset at the next general.alignment boundary, default 32);
  * Value::as_u64 / as_f32 / as_bool, gguf/mod.rs:36-80;
  * the MoE layer addressing of LlamaBackend::from_gguf, llama/mod.rs:569-607 (stacked
    blk.L.ffn_*_exps tensors, else split blk.L.ffn_*.E tensors), the element-count and
    byte-range checks of load_weight / pinned_weight (:320-381) and
    ExpertWeight::byte_range (:250-269).

Pinned by the reference's own GGUF tests (gguf/mod.rs:427-629), restated as
known-answer tests in tests/test_gguf.py, and by round trips through an independent
writer (garuda_amd.gguf.write_gguf).
"""
from __future__ import annotations

import struct

MAGIC = b"GGUF"


class GgufError(Exception):
    pass


def _bad(msg: str) -> GgufError:
    return GgufError("gguf: " + msg)


# gguf/mod.rs:227-244
def min_value_bytes(t: int) -> int:
    if t in (0, 1, 7):
        return 1
    if t in (2, 3):
        return 2
    if t in (4, 5, 6):
        return 4
    if t == 8:
        return 8
    if t == 9:
        return 12
    if t in (10, 11, 12):
        return 8
    return 1


class _Cursor:
    # gguf/mod.rs:113-178
    def __init__(self, buf: bytes):
        self.buf, self.pos = buf, 0

    def take(self, n: int) -> bytes:
        end = self.pos + n
        if end > len(self.buf):
            raise _bad(f"truncated: wanted {n} bytes at offset {self.pos}")
        b = self.buf[self.pos:end]
        self.pos = end
        return b

    def u(self, fmt: str) -> int:
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.u("<Q")
        if n > len(self.buf) - min(self.pos, len(self.buf)):
            raise _bad(f"string of {n} bytes overruns the {len(self.buf)}-byte file")
        b = self.take(n)
        try:
            return b.decode("utf-8")
        except UnicodeDecodeError as e:
            raise _bad(f"string is not valid UTF-8: {e}") from None

    # gguf/mod.rs:180-222; values are (type, payload)
    def value(self, t: int, depth: int):
        if depth > 8:
            raise _bad("metadata nests too deeply")
        fmts = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 10: "<Q", 11: "<q"}
        if t in fmts:
            return (t, self.u(fmts[t]))
        if t == 6:
            return (t, struct.unpack("<f", self.take(4))[0])
        if t == 7:
            return (t, self.u("<B") != 0)
        if t == 8:
            return (t, self.string())
        if t == 9:
            et = self.u("<I")
            n = self.u("<Q")
            remaining = max(0, len(self.buf) - self.pos)
            if n > remaining // max(min_value_bytes(et), 1):
                raise _bad(f"array of {n} elements overruns the {len(self.buf)}-byte file")
            return (t, (et, [self.value(et, depth + 1) for _ in range(n)]))
        if t == 12:
            return (t, struct.unpack("<d", self.take(8))[0])
        raise _bad(f"unknown metadata value type {t}")


def parse(data: bytes) -> dict:
    """{version, metadata {key: (type, payload)}, tensors [(name, dims, type, offset)],
    data_offset} or GgufError (gguf/mod.rs:247-324)."""
    c = _Cursor(bytes(data))
    magic = c.take(4)
    if magic != MAGIC:
        raise _bad(f"bad magic {list(magic)}, expected {list(MAGIC)}")
    version = c.u("<I")
    if not 2 <= version <= 3:
        raise _bad(f"unsupported version {version}")
    tensor_count = c.u("<Q")
    kv_count = c.u("<Q")
    remaining = len(c.buf) - c.pos
    if tensor_count > remaining // 24 or kv_count > remaining // 13:
        raise _bad(f"header claims {tensor_count} tensors and {kv_count} metadata entries, "
                   f"more than the remaining {remaining} bytes can describe")
    meta = {}
    for _ in range(kv_count):
        key = c.string()
        t = c.u("<I")
        meta[key] = c.value(t, 0)
    tensors = []
    for _ in range(tensor_count):
        name = c.string()
        n_dims = c.u("<I")
        if n_dims > 4:
            raise _bad(f"tensor '{name}' claims {n_dims} dimensions")
        dims = [c.u("<Q") for _ in range(n_dims)]
        t = c.u("<I")
        off = c.u("<Q")
        tensors.append((name, dims, t, off))
    a = as_u64(meta["general.alignment"]) if "general.alignment" in meta else None
    align = 32 if a is None else a
    if align == 0 or align & (align - 1):
        raise _bad(f"alignment {align} is not a power of two")
    data_offset = (c.pos + align - 1) // align * align
    return {"version": version, "metadata": dict(sorted(meta.items())), "tensors": tensors,
            "data_offset": data_offset}


# gguf/mod.rs:36-49
def as_u64(v):
    t, x = v
    if t in (0, 2, 4, 10):
        return x
    if t in (1, 3, 5, 11) and x >= 0:
        return x
    return None


# gguf/mod.rs:58-64 (f32 rounding left to the caller's comparison)
def as_f32(v):
    t, x = v
    if t in (6, 12):
        return x
    u = as_u64(v)
    return None if u is None else float(u)


# gguf/mod.rs:75-80
def as_bool(v):
    t, x = v
    if t == 7:
        return x
    u = as_u64(v)
    return None if u is None else u != 0


# quant/mod.rs:41-61
_LAYOUT = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144),
           13: (256, 176), 14: (256, 210)}


def byte_size(t: int, n: int):
    if t not in _LAYOUT or n % _LAYOUT[t][0]:
        return None
    e, b = _LAYOUT[t]
    return n // e * b


def _tensor(g, name):
    for t in g["tensors"]:  # Gguf::tensor: the first match
        if t[0] == name:
            return t
    return None


def _weight(g, file_len, name, rows, cols):
    # load_weight / pinned_weight, llama/mod.rs:320-381 -> (type, file start, nbytes)
    t = _tensor(g, name)
    if t is None:
        raise _bad(f"tensor '{name}' not found")
    n = 1
    for d in t[1]:
        n *= d
    if n != rows * cols:
        raise _bad(f"tensor '{name}' has {n} elements, expected {rows * cols}")
    nb = byte_size(t[2], n)
    if nb is None:
        raise _bad(f"tensor '{name}': type {t[2]} is not supported")
    start = g["data_offset"] + t[3]
    if start + nb > file_len:
        raise _bad(f"tensor '{name}' runs past the end of its buffer")
    return t[2], start, nb


def moe_dims(g):
    arch = g["metadata"].get("general.architecture")
    if arch is None or arch[0] != 8:
        raise _bad("no general.architecture")
    out = {}
    for key in ("embedding_length", "feed_forward_length", "block_count", "expert_count", "expert_used_count"):
        v = g["metadata"].get(f"{arch[1]}.{key}")
        u = None if v is None else as_u64(v)
        if u is None and key.startswith("expert"):
            u = 0  # LlamaConfig::from_gguf, llama/mod.rs:462-463: absent counts are 0
        if u is None:
            raise _bad(f"gguf is missing {arch[1]}.{key}")
        out[key] = u
    return out["embedding_length"], out["feed_forward_length"], out["expert_count"], out["expert_used_count"], \
        out["block_count"]


def layer(g, file_len: int, l: int) -> dict:
    """The feed-forward tensors of layer l (llama/mod.rs:569-613): {router: (type, start,
    nbytes), layout: 'stacked'|'split', gate/up/down: (type, [start per expert], bytes per
    expert)}; a dense FFN (Ffn::Dense) is layout 'dense', one expert, top-1, router None."""
    d, f, ne, k, nl = moe_dims(g)
    if l >= nl:
        raise _bad(f"layer {l} of a {nl}-layer model")
    p = lambda name: f"blk.{l}.{name}.weight"  # noqa: E731
    pe = lambda name, e: f"blk.{l}.{name}.{e}.weight"  # noqa: E731
    shapes = {"gate": ("ffn_gate", f, d), "up": ("ffn_up", f, d), "down": ("ffn_down", d, f)}
    moe = ne > 0 and (_tensor(g, p("ffn_gate_exps")) is not None or _tensor(g, pe("ffn_gate", 0)) is not None)
    if not moe:
        if _tensor(g, p("ffn_gate")) is None:
            raise _bad(f"layer {l} has no feed-forward tensors")
        out = {"d": d, "f": f, "ne": 1, "k": 1, "router": None, "layout": "dense"}
        for key, (base, rows, cols) in shapes.items():
            t, start, nb = _weight(g, file_len, p(base), rows, cols)
            out[key] = (t, [start], nb)
        return out
    out = {"d": d, "f": f, "ne": ne, "k": k, "router": _weight(g, file_len, p("ffn_gate_inp"), ne, d)}
    if ne > 0 and _tensor(g, p("ffn_gate_exps")) is not None:
        out["layout"] = "stacked"
        for key, (base, rows, cols) in shapes.items():
            t, start, nb = _weight(g, file_len, p(base + "_exps"), ne * rows, cols)
            per = nb // ne  # ExpertWeight::byte_range: expert e at start + e*rows*row_bytes
            out[key] = (t, [start + e * per for e in range(ne)], per)
    elif ne > 0 and _tensor(g, pe("ffn_gate", 0)) is not None:
        out["layout"] = "split"
        for key, (base, rows, cols) in shapes.items():
            ws = [_weight(g, file_len, pe(base, e), rows, cols) for e in range(ne)]
            out[key] = (ws[0][0], [w[1] for w in ws], ws[0][2])
    else:
        raise _bad(f"layer {l} has no expert tensors")
    return out
