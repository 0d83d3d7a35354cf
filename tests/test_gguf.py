"""GGUF reader (garuda_amd/csrc/gmoe_gguf.cpp through the C-ABI) against the oracle's
restatement of gguf::Gguf (oracle/gguf.py), and both against the reference's own GGUF
tests (garuda/src/gguf/mod.rs:427-629), restated here as known-answer tests.

Host code only: no GPU.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import gguf as gg
from oracle import gguf as OG
from oracle import oracle as O


# ---- the reference test module's Builder (gguf/mod.rs:431-501), restated ----
class RefBuilder:
    def __init__(self):
        self.kv, self.kv_count, self.tensors, self.tensor_count = bytearray(), 0, bytearray(), 0

    @staticmethod
    def _str(out, s):
        b = s.encode()
        out += struct.pack("<Q", len(b)) + b

    def kv_string(self, key, value):
        self._str(self.kv, key)
        self.kv += struct.pack("<I", 8)
        self._str(self.kv, value)
        self.kv_count += 1
        return self

    def kv_u32(self, key, value):
        self._str(self.kv, key)
        self.kv += struct.pack("<II", 4, value)
        self.kv_count += 1
        return self

    def kv_str_array(self, key, values):
        self._str(self.kv, key)
        self.kv += struct.pack("<IIQ", 9, 8, len(values))
        for v in values:
            self._str(self.kv, v)
        self.kv_count += 1
        return self

    def tensor(self, name, dims, ggml_type, offset):
        self._str(self.tensors, name)
        self.tensors += struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        self.tensors += struct.pack("<IQ", ggml_type, offset)
        self.tensor_count += 1
        return self

    def build(self):
        out = bytearray(b"GGUF") + struct.pack("<IQQ", 3, self.tensor_count, self.kv_count)
        out += self.kv + self.tensors
        out += bytes(-len(out) % 32)
        out += bytes(64)  # tensor data
        return bytes(out)


def mixtral_like():  # gguf/mod.rs:503-513
    return (RefBuilder()
            .kv_string("general.architecture", "llama")
            .kv_u32("llama.expert_count", 8)
            .kv_u32("llama.expert_used_count", 2)
            .kv_u32("llama.block_count", 32)
            .kv_str_array("tokenizer.ggml.tokens", ["<unk>", "<s>", "hello"])
            .tensor("token_embd.weight", [4096, 32000], 12, 0)
            .tensor("blk.0.ffn_gate_exps.weight", [4096, 14336, 8], 12, 1024)
            .build())


def lib_parse(data):
    return G.Gguf.parse(data)


def lib_ok(data) -> bool:
    try:
        lib_parse(data).close()
        return True
    except G.ModelError:
        return False


def oracle_ok(data) -> bool:
    try:
        OG.parse(data)
        return True
    except OG.GgufError:
        return False


def _norm(t, x):
    """(type, payload) with floats as their bits, so NaNs compare."""
    if t == gg.F32:
        return (t, struct.pack("<f", x))
    if t == gg.F64:
        return (t, struct.pack("<d", x))
    if t == gg.ARRAY:
        et, items = x
        return (t, (et, [_norm(*i) for i in items]))
    return (t, x)


def lib_view(g: G.Gguf):
    def conv(v: G.Value):
        if v.type == gg.ARRAY:
            return (v.type, (v.elem_type, [conv(i) for i in v.value]))
        return _norm(v.type, v.value)
    meta = {k: conv(v) for k, v in g.metadata.items()}
    tensors = [(t.name, t.dims, t.ggml_type, t.offset) for t in g.tensors]
    return {"version": g.version, "metadata": meta, "tensors": tensors, "data_offset": g.data_offset}


def oracle_view(data):
    o = OG.parse(data)
    o["metadata"] = {k: _norm(*v) for k, v in o["metadata"].items()}
    return o


# ---- the reference's tests, on both readers ----

def test_parses_a_real_looking_header():  # gguf/mod.rs:515-525
    g = lib_parse(mixtral_like())
    assert g.version == 3
    assert g.architecture() == "llama"
    assert g.expert_count() == 8
    assert g.expert_used_count() == 2
    assert len(g.tensors) == 2
    assert g.data_offset % 32 == 0
    o = OG.parse(mixtral_like())
    assert (o["version"], len(o["tensors"]), o["data_offset"]) == (3, 2, g.data_offset)
    assert OG.as_u64(o["metadata"]["llama.expert_count"]) == 8


def test_reads_tensor_descriptors():  # gguf/mod.rs:527-539
    g = lib_parse(mixtral_like())
    t = g.tensor("blk.0.ffn_gate_exps.weight")
    assert t.dims == [4096, 14336, 8]
    assert t.ggml_type == 12
    assert t.offset == 1024
    assert t.n_elements() == 4096 * 14336 * 8
    assert t.data == 0  # its 33 MB are not in this 64-byte data section
    assert g.tensor("nonexistent") is None
    o = OG.parse(mixtral_like())
    assert o["tensors"][1] == ("blk.0.ffn_gate_exps.weight", [4096, 14336, 8], 12, 1024)


def test_reads_arrays():  # gguf/mod.rs:541-549
    g = lib_parse(mixtral_like())
    tokens = g.metadata["tokenizer.ggml.tokens"].as_array()
    assert len(tokens) == 3
    assert tokens[2].as_str() == "hello"
    assert OG.parse(mixtral_like())["metadata"]["tokenizer.ggml.tokens"][1][1][2] == (8, "hello")


@pytest.mark.parametrize("data", [b"not a gguf file at all", b"", bytes(3)])
def test_rejects_a_non_gguf_file(data):  # gguf/mod.rs:551-556
    assert not lib_ok(data)
    assert not oracle_ok(data)


def test_truncation_anywhere_is_an_error_not_a_crash():  # gguf/mod.rs:558-566
    full = mixtral_like()
    for cut in range(len(full) + 1):
        assert lib_ok(full[:cut]) == oracle_ok(full[:cut]), f"readers disagree at cut {cut}"
    assert not lib_ok(full[:30])
    assert lib_ok(full)


def test_a_lying_length_field_does_not_cause_a_huge_allocation():  # gguf/mod.rs:568-579
    data = b"GGUF" + struct.pack("<IQQQ", 3, 0, 1, (1 << 64) - 1)
    with pytest.raises(G.ModelError):
        lib_parse(data)
    assert not oracle_ok(data)


def test_absurd_header_counts_are_rejected():  # gguf/mod.rs:581-589
    data = b"GGUF" + struct.pack("<IQQ", 3, (1 << 64) - 1, 0)
    assert not lib_ok(data) and not oracle_ok(data)


def test_a_count_the_remaining_bytes_cannot_describe_is_rejected():  # gguf/mod.rs:591-614
    body = bytes(4096)
    tensors = b"GGUF" + struct.pack("<IQQ", 3, 2000, 0) + body
    kvs = b"GGUF" + struct.pack("<IQQ", 3, 0, 2000) + body
    for data in (tensors, kvs):
        assert not lib_ok(data) and not oracle_ok(data)


def test_an_arrays_declared_length_is_bounded_by_its_element_size():  # gguf/mod.rs:616-632
    data = (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 4) + b"toks" +
            struct.pack("<IIQ", 9, 10, 900) + bytes(1000))
    with pytest.raises(G.ModelError, match="overruns"):
        lib_parse(data)
    with pytest.raises(OG.GgufError, match="overruns"):
        OG.parse(data)


def test_as_bool_accepts_both_the_bool_and_integer_encodings():  # gguf/mod.rs:634-641
    assert G.Value(gg.BOOL, True).as_bool() is True
    assert G.Value(gg.BOOL, False).as_bool() is False
    assert G.Value(gg.U32, 1).as_bool() is True
    assert G.Value(gg.U8, 0).as_bool() is False
    assert G.Value(gg.STRING, "yes").as_bool() is None
    assert OG.as_bool((gg.U32, 1)) is True and OG.as_bool((gg.STRING, "yes")) is None


def test_an_unsupported_version_is_rejected():  # gguf/mod.rs:643-648
    data = bytearray(mixtral_like())
    data[4:8] = struct.pack("<I", 99)
    assert not lib_ok(bytes(data)) and not oracle_ok(bytes(data))
    data[4:8] = struct.pack("<I", 2)
    assert lib_ok(bytes(data)) and oracle_ok(bytes(data))


# ---- more of the format, on both readers ----

def rich_file(alignment=None):
    """Every value type, a nested array, a repeated key and two tensors with data."""
    meta = [("general.architecture", gg.STRING, "llama"),
            ("a.u8", gg.U8, 200), ("a.i8", gg.I8, -5), ("a.u16", gg.U16, 65000), ("a.i16", gg.I16, -300),
            ("a.u32", gg.U32, 4000000000), ("a.i32", gg.I32, -7), ("a.f32", gg.F32, 1.5),
            ("a.bool", gg.BOOL, True), ("a.str", gg.STRING, "héllo ☃"),
            ("a.u64", gg.U64, (1 << 64) - 2), ("a.i64", gg.I64, -(1 << 40)), ("a.f64", gg.F64, -2.25),
            ("a.arr", gg.ARRAY, (gg.I32, [1, -2, 3])),
            ("a.nested", gg.ARRAY, (gg.ARRAY, [(gg.U8, [1, 2]), (gg.U8, [])])),
            ("a.u8", gg.U8, 7)]  # repeated: the last value stays
    if alignment is not None:
        meta.append(("general.alignment", gg.U32, alignment))
    tensors = [("x.weight", [8, 2], G.F32, np.arange(16, dtype=np.float32).tobytes()),
               ("y.weight", [32], G.Q8_0, bytes(34))]
    return gg.write_gguf(meta, tensors, alignment=alignment or 32)


def test_every_value_type_matches_the_oracle():
    data = rich_file()
    assert lib_view(lib_parse(data)) == oracle_view(data)
    g = lib_parse(data)
    assert g.get("a.u8").value == 7 and len(g.metadata) == 15
    assert g.get("a.i32").as_u64() is None and g.get("a.u32").as_u64() == 4000000000
    assert g.get("a.f32").as_f32() == 1.5 and g.get("a.u16").as_f32() == 65000.0
    assert g.get("a.str").as_str() == "héllo ☃"
    assert g.get("missing") is None
    x = g.tensor("x.weight")
    assert np.array_equal(np.frombuffer(x.bytes().tobytes(), dtype=np.float32), np.arange(16, dtype=np.float32))


@pytest.mark.parametrize("alignment", [1, 64, 4096])
def test_alignment_sets_the_data_offset(alignment):
    data = rich_file(alignment)
    g = lib_parse(data)
    assert g.data_offset % alignment == 0 and g.data_offset == OG.parse(data)["data_offset"]
    assert np.array_equal(np.frombuffer(g.tensor("x.weight").bytes().tobytes(), dtype=np.float32),
                          np.arange(16, dtype=np.float32))


def test_bad_alignments():
    for key_t, v in ((gg.U32, 48), (gg.U32, 0)):
        data = gg.write_gguf([("general.alignment", key_t, v)], [], alignment=64)
        assert not lib_ok(data) and not oracle_ok(data)
    # a negative alignment is no integer to as_u64: the default 32 applies
    data = gg.write_gguf([("general.alignment", gg.I32, -64)], [])
    assert lib_parse(data).data_offset % 32 == 0 and oracle_ok(data)


def test_strings_must_be_utf8():
    for bad in (b"\xff", b"\xc0\x80", b"\xed\xa0\x80", b"\xf4\x90\x80\x80", b"ab\xe2\x82"):
        data = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", len(bad)) + bad + \
            struct.pack("<IB", 0, 1) + bytes(16)
        assert not lib_ok(data) and not oracle_ok(data), bad


def test_nesting_depth_is_capped():
    def nested(depth):  # an array nesting `depth` arrays, innermost empty
        v = struct.pack("<IQ", 0, 0)  # empty array of u8
        for _ in range(depth):
            v = struct.pack("<IQ", 9, 1) + v
        return b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 9) + v + \
            bytes(32)
    assert lib_ok(nested(8)) and oracle_ok(nested(8))
    assert not lib_ok(nested(9)) and not oracle_ok(nested(9))


def test_unknown_types_and_dims():
    unk = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13) + bytes(32)
    assert not lib_ok(unk) and not oracle_ok(unk)
    empty_unknown_array = (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" +
                           struct.pack("<IIQ", 9, 13, 0) + bytes(32))
    assert lib_ok(empty_unknown_array) and oracle_ok(empty_unknown_array)
    five = RefBuilder().tensor("t", [1, 1, 1, 1, 1], 0, 0).build()
    assert not lib_ok(five) and not oracle_ok(five)


def test_mutated_files_agree_with_the_oracle():
    base = rich_file()
    rng = np.random.default_rng(7)
    accepted = 0
    for i in range(400):
        data = bytearray(base)
        kind = i % 3
        if kind == 0:  # flip bytes
            for _ in range(int(rng.integers(1, 4))):
                data[int(rng.integers(0, len(data)))] ^= int(rng.integers(1, 256))
        elif kind == 1:  # overwrite a length-sized field with a random u64
            at = int(rng.integers(0, len(data) - 8))
            data[at:at + 8] = struct.pack("<Q", int(rng.integers(0, 1 << 20)))
        else:  # truncate and flip
            data = data[:int(rng.integers(0, len(data)))]
            if data:
                data[int(rng.integers(0, len(data)))] ^= 0x55
        data = bytes(data)
        lo, oo = lib_ok(data), oracle_ok(data)
        assert lo == oo, f"mutation {i}: library {lo}, oracle {oo}"
        if lo:
            accepted += 1
            assert lib_view(lib_parse(data)) == oracle_view(data), f"mutation {i}"
    assert accepted > 20


# ---- MoE layer addressing (llama/mod.rs:569-607, :250-269) ----

def moe_file(layout="stacked", d=256, f=512, ne=4, nl=2, qts=(G.Q4_K, G.Q4_K, G.Q8_0), router_t=G.F32,
             seed=0, drop=None, bad_elems=None, split_types=None):
    """A small MoE checkpoint; the same numbers in either layout. `drop` omits a tensor,
    `bad_elems` gives a tensor a wrong shape."""
    rng = np.random.default_rng(seed)
    meta = [("general.architecture", gg.STRING, "llama"), ("llama.embedding_length", gg.U32, d),
            ("llama.feed_forward_length", gg.U32, f), ("llama.block_count", gg.U32, nl),
            ("llama.expert_count", gg.U32, ne), ("llama.expert_used_count", gg.U32, 2),
            ("tokenizer.ggml.tokens", gg.ARRAY, (gg.STRING, ["a", "b"]))]
    tensors = []
    for l in range(nl):
        r = rng.normal(0, 0.02, (ne, d)).astype(np.float32)
        rb = r.tobytes() if router_t == G.F32 else r.astype(np.float16).tobytes()
        tensors.append((f"blk.{l}.ffn_gate_inp.weight", [d, ne], router_t, rb))
        for (base, rows, cols), qt in zip((("ffn_gate", f, d), ("ffn_up", f, d), ("ffn_down", d, f)), qts):
            raw = G.quantize(qt, rng.normal(0, 0.02, ne * rows * cols).astype(np.float32)).tobytes()
            if layout == "stacked":
                tensors.append((f"blk.{l}.{base}_exps.weight", [cols, rows, ne], qt, raw))
            else:
                per = len(raw) // ne
                for e in range(ne):
                    et = qt
                    chunk = raw[e * per:(e + 1) * per]
                    if split_types and (l, base, e) in split_types:
                        et = split_types[(l, base, e)]
                        chunk = G.quantize(et, np.zeros(rows * cols, np.float32)).tobytes()
                    tensors.append((f"blk.{l}.{base}.{e}.weight", [cols, rows], et, chunk))
    if drop:
        tensors = [t for t in tensors if t[0] != drop]
    if bad_elems:
        tensors = [(n, [dm[0] // 2] + dm[1:], qt, raw[:len(raw) // 2]) if n == bad_elems else (n, dm, qt, raw)
                   for n, dm, qt, raw in tensors]
    return gg.write_gguf(meta, tensors)


def _desc(g, layer):
    from garuda_amd._lib import GmoeLayerDesc, lib
    import ctypes as C
    desc = GmoeLayerDesc()
    G.moe._check(lib().gmoe_gguf_layer_desc(g.handle, layer, 0, 0, 0, C.byref(desc)))
    return desc


@pytest.mark.parametrize("layout", ["stacked", "split"])
def test_layer_desc_points_at_the_oracles_bytes(layout):
    data = moe_file(layout)
    g = lib_parse(data)
    base = g._keep.ctypes.data
    o = OG.parse(data)
    for l in range(2):
        want = OG.layer(o, len(data), l)
        desc = _desc(g, l)
        assert (desc.d_model, desc.d_ff, desc.n_experts, desc.top_k) == (256, 512, 4, 2)
        assert desc.router[0] == np.frombuffer(data, np.float32, 1, want["router"][1])[0]
        assert C_addr(desc.router) - base == want["router"][1]
        for name in ("gate", "up", "down"):
            t = getattr(desc, name)
            qt, starts, per = want[name]
            assert t.qtype == qt
            if layout == "stacked":
                assert t.layout == G.moe.LAYOUT_STACKED and t.data - base == starts[0]
            else:
                assert t.layout == G.moe.LAYOUT_SPLIT
                assert [t.experts[e] - base for e in range(4)] == starts
        for e in range(4):
            rngs = g.expert_ranges(l, e)
            assert rngs == [(want[n][1][e], want[n][2]) for n in ("gate", "up", "down")]


def C_addr(p):
    import ctypes as C
    return C.cast(p, C.c_void_p).value


def test_both_layouts_hold_the_same_expert_bytes():
    a, b = moe_file("stacked"), moe_file("split")
    ga, gb = lib_parse(a), lib_parse(b)
    for l in range(2):
        for e in range(4):
            for (oa, la), (ob, lb) in zip(ga.expert_ranges(l, e), gb.expert_ranges(l, e)):
                assert la == lb and a[oa:oa + la] == b[ob:ob + lb]


def test_f16_router_is_widened_exactly():
    data = moe_file(router_t=G.F16)
    g = lib_parse(data)
    o = OG.parse(data)
    want = OG.layer(o, len(data), 1)
    r16 = np.frombuffer(data, np.float16, 256 * 4, want["router"][1])
    desc = _desc(g, 1)
    got = np.ctypeslib.as_array(desc.router, shape=(4 * 256,))
    assert np.array_equal(got, r16.astype(np.float32))


def test_layer_desc_refusals():
    cases = [
        (moe_file(drop="blk.1.ffn_up_exps.weight"), 1, "not found"),
        (moe_file(bad_elems="blk.0.ffn_down_exps.weight"), 0, "elements, expected"),
        (moe_file("split", split_types={(0, "ffn_up", 2): G.Q6_K}), 0, "one type per matrix"),
        (moe_file(), 2, "layer 2 of a 2-layer model"),
        (moe_file(drop="blk.0.ffn_gate_exps.weight"), 0, "no feed-forward tensors"),
        (moe_file(drop="blk.0.ffn_gate_inp.weight"), 0, "not found"),
    ]
    for data, layer, msg in cases:
        g = lib_parse(data)
        with pytest.raises((G.ModelError, G.InferenceError), match=msg):
            _desc(g, layer)
    # a file cut inside layer 1's data: layer 0 still loads, layer 1 is refused
    data = moe_file()
    o = OG.parse(data)
    cut = OG.layer(o, len(data), 1)["down"][1][0] + 10
    g = lib_parse(data[:cut])
    _desc(g, 0)
    with pytest.raises(G.ModelError, match="past the end"):
        _desc(g, 1)
    with pytest.raises(OG.GgufError, match="past the end"):
        OG.layer(OG.parse(data[:cut]), cut, 1)


def test_open_maps_a_file(tmp_path):
    data = moe_file()
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    with G.Gguf.open(p) as g:
        assert g.file_bytes == len(data) and g.expert_count() == 4
        t = g.tensor("blk.0.ffn_gate_exps.weight")
        assert t.bytes().tobytes() == data[g.data_offset + t.offset:g.data_offset + t.offset + t.nbytes]
    with pytest.raises(G.ModelError, match="cannot open"):
        G.Gguf.open(tmp_path / "missing.gguf")


def test_streamed_writer_matches(tmp_path):
    meta = [("general.architecture", gg.STRING, "x"), ("general.alignment", gg.U32, 64)]
    tensors = [("a", [8], G.F32, np.arange(8, dtype=np.float32)), ("b", [32], G.Q8_0, np.zeros(34, np.uint8)),
               ("c", [256], G.Q4_K, G.quantize(G.Q4_K, np.linspace(-1, 1, 256, dtype=np.float32)))]
    n = gg.write_gguf_file(tmp_path / "w.gguf", meta, tensors, alignment=64)
    data = (tmp_path / "w.gguf").read_bytes()
    assert n == len(data) and data == gg.write_gguf(meta, tensors, alignment=64)
    g = lib_parse(data)
    assert g.data_offset % 64 == 0 and all(t.offset % 64 == 0 for t in g.tensors)
    assert g.tensor("c").bytes().tobytes() == tensors[2][3].tobytes()


# ---- dense feed-forward layers (Ffn::Dense, llama/mod.rs:590-613, :913-920) ----

def dense_file(d=256, f=512, ne=4, with_counts=True, seed=1):
    """Layer 0 MoE (stacked), layer 1 dense (blk.1.ffn_gate/up/down); with_counts False:
    no expert counts at all, every layer dense."""
    rng = np.random.default_rng(seed)
    meta = [("general.architecture", gg.STRING, "llama"), ("llama.embedding_length", gg.U32, d),
            ("llama.feed_forward_length", gg.U32, f), ("llama.block_count", gg.U32, 2)]
    if with_counts:
        meta += [("llama.expert_count", gg.U32, ne), ("llama.expert_used_count", gg.U32, 2)]
    tensors = []
    for l in range(2):
        moe = with_counts and l == 0
        if moe:
            tensors.append((f"blk.{l}.ffn_gate_inp.weight", [d, ne], G.F32,
                            rng.normal(0, 0.02, (ne, d)).astype(np.float32).tobytes()))
        for base, rows, cols in (("ffn_gate", f, d), ("ffn_up", f, d), ("ffn_down", d, f)):
            m = ne if moe else 1
            raw = G.quantize(G.Q4_K, rng.normal(0, 0.02, m * rows * cols).astype(np.float32)).tobytes()
            name = f"blk.{l}.{base}_exps.weight" if moe else f"blk.{l}.{base}.weight"
            tensors.append((name, [cols, rows, ne] if moe else [cols, rows], G.Q4_K, raw))
    return gg.write_gguf(meta, tensors)


@pytest.mark.parametrize("with_counts", [True, False])
def test_a_dense_layer_is_one_expert_of_weight_one(with_counts):
    data = dense_file(with_counts=with_counts)
    g = lib_parse(data)
    base = g._keep.ctypes.data
    o = OG.parse(data)
    want = OG.layer(o, len(data), 1)
    assert want["layout"] == "dense" and (want["ne"], want["k"]) == (1, 1) and want["router"] is None
    desc = _desc(g, 1)
    assert (desc.d_model, desc.d_ff, desc.n_experts, desc.top_k) == (256, 512, 1, 1)
    assert not np.ctypeslib.as_array(desc.router, shape=(256,)).any()  # a zero router: weight 1 under any gating
    for name in ("gate", "up", "down"):
        t = getattr(desc, name)
        qt, starts, per = want[name]
        assert t.qtype == qt and t.layout == G.moe.LAYOUT_STACKED and t.data - base == starts[0]
    if with_counts:
        assert _desc(g, 0).n_experts == 4 and OG.layer(o, len(data), 0)["layout"] == "stacked"
    for kind in range(4):  # every gating of a single logit gives weight 1 exactly
        ids, w = O.gate(kind, np.array([0.0], np.float32), 1)
        assert ids.tolist() == [0] and w.tolist() == [1.0]
