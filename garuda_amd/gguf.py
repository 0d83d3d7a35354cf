"""GGUF checkpoints: the reference's `gguf::Gguf` (garuda/src/gguf/mod.rs), parsed by the
library's C++ reader (gmoe_gguf_* in include/garuda_moe.h), and a writer for building
synthetic checkpoints.

`Gguf.open(path)` maps the file read-only; `Gguf.parse(data)` reads a bytes-like
object. The attributes and accessors mirror the reference's: `version`, `metadata`
(key -> `Value`), `tensors` (`TensorInfo` in file order), `data_offset`,
`architecture()`, `expert_count()`, `expert_used_count()`, `get()`, `arch_u64()`,
`arch_f32()`, `tensor()`. A malformed file raises `ModelError` with the reference's
message texts; a missing key or tensor gives `None`, as the reference's `Option`s do.

`MoeLayer.from_gguf(dev, gguf, layer)` registers an MoE layer straight from the file's
bytes (llama/mod.rs:569-607); `Gguf.expert_ranges()` gives an expert's file byte ranges
(llama/mod.rs:250-269, :664-682).
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass, field

import numpy as np

from ._lib import GmoeGgufHeader, GmoeGgufTensorInfo, GmoeGgufValue, lib
from .moe import NotFoundError, _check, byte_size

# metadata value types (gguf/mod.rs:181-221)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SIGNED = {I8: 8, I16: 16, I32: 32, I64: 64}


@dataclass(frozen=True)
class Value:
    """A metadata value (gguf::Value, gguf/mod.rs:18-33): its GGUF type id and payload
    (int, float, bool, str, or a list of Values)."""

    type: int
    value: object
    elem_type: int = 0

    # gguf/mod.rs:36-49
    def as_u64(self):
        if self.type in (U8, U16, U32, U64):
            return self.value
        if self.type in _SIGNED and self.value >= 0:
            return self.value
        return None

    def as_str(self):
        return self.value if self.type == STRING else None

    # gguf/mod.rs:58-64
    def as_f32(self):
        if self.type in (F32, F64):
            return float(np.float32(self.value))
        u = self.as_u64()
        return None if u is None else float(np.float32(u))

    def as_array(self):
        return self.value if self.type == ARRAY else None

    # gguf/mod.rs:75-80
    def as_bool(self):
        if self.type == BOOL:
            return bool(self.value)
        u = self.as_u64()
        return None if u is None else u != 0


@dataclass
class TensorInfo:
    """A tensor descriptor (gguf::TensorInfo, gguf/mod.rs:83-97); `nbytes` and `data`
    (the address of its bytes in the file, 0 if they run past the end) are extras."""

    name: str
    dims: list
    ggml_type: int
    offset: int
    nbytes: int = 0
    data: int = 0
    _owner: object = field(default=None, repr=False, compare=False)

    def n_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n

    def bytes(self) -> np.ndarray:
        """The tensor's raw bytes inside the file (a read-only view; the checkpoint must
        stay open while it is used)."""
        if not self.data:
            raise NotFoundError(f"gguf: tensor '{self.name}' runs past the end of the file")
        buf = (C.c_uint8 * self.nbytes).from_address(self.data)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a


def _value(v: GmoeGgufValue, h=None) -> Value:
    t = v.type
    if t == STRING:
        return Value(t, C.string_at(v.str, v.len).decode("utf-8"))
    if t in (F32, F64):
        return Value(t, float(v.f))
    if t == BOOL:
        return Value(t, bool(v.u))
    if t in _SIGNED:
        x = v.u & ((1 << 64) - 1)
        return Value(t, x - (1 << 64) if x >> 63 else x)
    if t == ARRAY:
        items = []
        for i in range(v.len):
            iv = GmoeGgufValue()
            _check(lib().gmoe_gguf_array_item(h, C.byref(v), i, C.byref(iv)))
            items.append(_value(iv, h))
        return Value(t, items, v.elem_type)
    return Value(t, int(v.u))


class Gguf:
    """A parsed GGUF file (gguf::Gguf, gguf/mod.rs:100-106, :246-396)."""

    def __init__(self, handle, keep=None):
        self._h = handle
        self._keep = keep
        hd = GmoeGgufHeader()
        _check(lib().gmoe_gguf_get_header(self._h, C.byref(hd)))
        self.version = hd.version
        self.data_offset = hd.data_offset
        self.file_bytes = hd.file_bytes
        self._n_tensors, self._n_keys = hd.n_tensors, hd.n_keys
        self._meta = None
        self._tensors = None

    @classmethod
    def open(cls, path) -> "Gguf":
        h = C.c_void_p()
        _check(lib().gmoe_gguf_open(str(path).encode(), C.byref(h)))
        return cls(h)

    @classmethod
    def parse(cls, data) -> "Gguf":
        buf = np.frombuffer(bytes(data), dtype=np.uint8) if not isinstance(data, np.ndarray) else data
        buf = np.ascontiguousarray(buf, dtype=np.uint8)
        h = C.c_void_p()
        _check(lib().gmoe_gguf_parse(buf.ctypes.data if buf.size else None, buf.size, C.byref(h)))
        return cls(h, keep=buf)

    @property
    def handle(self):
        if self._h is None:
            raise ValueError("GGUF file is closed")
        return self._h

    def close(self) -> None:
        if self._h is not None:
            lib().gmoe_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- metadata ----
    def _get(self, key: str):
        v = GmoeGgufValue()
        try:
            _check(lib().gmoe_gguf_get_value(self.handle, key.encode(), C.byref(v)))
        except NotFoundError:
            return None
        return _value(v, self.handle)

    @property
    def metadata(self) -> dict:
        if self._meta is None:
            keys = []
            for i in range(self._n_keys):
                k = C.c_char_p()
                _check(lib().gmoe_gguf_key_at(self.handle, i, C.byref(k)))
                keys.append(k.value.decode("utf-8"))
            self._meta = {k: self._get(k) for k in keys}
        return self._meta

    def get(self, key: str):
        """A metadata value keyed exactly, or None (gguf/mod.rs:362-365)."""
        return self._get(key)

    def architecture(self):
        v = self.get("general.architecture")
        return None if v is None else v.as_str()

    def _arch(self, suffix: str):
        a = self.architecture()
        return None if a is None else self.get(f"{a}.{suffix}")

    def arch_u64(self, suffix: str):
        v = self._arch(suffix)
        return None if v is None else v.as_u64()

    def arch_f32(self, suffix: str):
        v = self._arch(suffix)
        return None if v is None else v.as_f32()

    def expert_count(self):
        return self.arch_u64("expert_count")

    def expert_used_count(self):
        return self.arch_u64("expert_used_count")

    # ---- tensors ----
    @staticmethod
    def _info(ti: GmoeGgufTensorInfo, owner) -> TensorInfo:
        return TensorInfo(ti.name.decode("utf-8"), [int(ti.dims[i]) for i in range(ti.n_dims)], ti.qtype,
                          ti.offset, ti.nbytes, ti.data or 0, owner)

    @property
    def tensors(self) -> list:
        if self._tensors is None:
            out = []
            for i in range(self._n_tensors):
                ti = GmoeGgufTensorInfo()
                _check(lib().gmoe_gguf_tensor_at(self.handle, i, C.byref(ti)))
                out.append(self._info(ti, self))
            self._tensors = out
        return self._tensors

    def tensor(self, name: str):
        """The first tensor called `name`, or None (gguf/mod.rs:393-395)."""
        ti = GmoeGgufTensorInfo()
        try:
            _check(lib().gmoe_gguf_find_tensor(self.handle, name.encode(), C.byref(ti)))
        except NotFoundError:
            return None
        return self._info(ti, self)

    def expert_ranges(self, layer: int, expert: int):
        """[(offset, length)] of the expert's gate, up and down bytes in the file."""
        off, ln = (C.c_uint64 * 3)(), (C.c_uint64 * 3)()
        _check(lib().gmoe_gguf_expert_ranges(self.handle, layer, expert, off, ln))
        return [(int(off[i]), int(ln[i])) for i in range(3)]


# ---------------------------------------------------------------------------------
# Writer: the GGUF v2/v3 container (https://github.com/ggml-org/ggml/blob/master/docs/gguf.md),
# for synthetic checkpoints. Values are (type, payload); arrays are (ARRAY, (elem_type, items)).
# ---------------------------------------------------------------------------------
_PACK = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
         U64: "<Q", I64: "<q", F64: "<d"}


def _put_str(out: bytearray, s: str) -> None:
    b = s.encode("utf-8")
    out += struct.pack("<Q", len(b)) + b


def _put_value(out: bytearray, t: int, v) -> None:
    if t == STRING:
        _put_str(out, v)
    elif t == ARRAY:
        et, items = v
        out += struct.pack("<IQ", et, len(items))
        for x in items:
            _put_value(out, et, x)
    else:
        out += struct.pack(_PACK[t], int(v) if t == BOOL else v)


def _layout(metadata, tensors, version: int, alignment: int):
    """(header bytes up to the data section, tensor offsets, data section size)."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, t, v in metadata:
        _put_str(out, key)
        out += struct.pack("<I", t)
        _put_value(out, t, v)
    offs, cur = [], 0
    for name, dims, qt, raw in tensors:
        cur = (cur + alignment - 1) // alignment * alignment
        offs.append(cur)
        n = 1
        for d in dims:
            n *= d
        nb = memoryview(raw).nbytes
        if nb != byte_size(qt, n):
            raise ValueError(f"tensor {name}: {nb} bytes for {n} elements of type {qt}")
        cur += nb
    for (name, dims, qt, raw), off in zip(tensors, offs):
        _put_str(out, name)
        out += struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", qt, off)
    out += bytes(-len(out) % alignment)
    return bytes(out), offs, (cur + alignment - 1) // alignment * alignment


def write_gguf(metadata, tensors, version: int = 3, alignment: int = 32) -> bytes:
    """A GGUF file: `metadata` is [(key, type, value)], `tensors` is
    [(name, dims, ggml_type, raw bytes)] with dims in ggml order (row length first).
    Tensor data is laid out in order, each tensor at the next `alignment` boundary of
    the data section, which starts at the next boundary after the descriptors."""
    head, offs, size = _layout(metadata, tensors, version, alignment)
    data = bytearray(size)
    for (_, _, _, raw), off in zip(tensors, offs):
        b = memoryview(raw).cast("B")
        data[off:off + b.nbytes] = b
    return head + bytes(data)


def write_gguf_file(path, metadata, tensors, version: int = 3, alignment: int = 32) -> int:
    """write_gguf streamed to `path` tensor by tensor (raw may be any buffer, e.g. a numpy
    array); returns the file size."""
    head, offs, size = _layout(metadata, tensors, version, alignment)
    with open(path, "wb") as fh:
        fh.write(head)
        at = 0
        for (_, _, _, raw), off in zip(tensors, offs):
            b = memoryview(raw).cast("B")
            fh.write(bytes(off - at))
            fh.write(b)
            at = off + b.nbytes
        fh.write(bytes(size - at))
    return len(head) + size
