"""ctypes wrapper of oracle/liboracle.so — the CPU restatement of the reference path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product never loads it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

F32, F16, Q4_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 10, 11, 12, 13, 14
INT8_TYPES = (Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K)
ALL_TYPES = (F32, F16, Q4_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K)

f32p, u32p, i32p, i8p, u8p = (C.POINTER(C.c_float), C.POINTER(C.c_uint32), C.POINTER(C.c_int32),
                              C.POINTER(C.c_int8), C.POINTER(C.c_uint8))
sz = C.c_size_t


class MoeLayerC(C.Structure):
    _fields_ = [
        ("d", C.c_int), ("f", C.c_int), ("ne", C.c_int), ("k", C.c_int),
        ("gating", C.c_int), ("combine", C.c_int), ("packed", C.c_int),
        ("router", f32p), ("qt_gate", C.c_uint32), ("qt_up", C.c_uint32), ("qt_down", C.c_uint32),
        ("gate", u8p), ("up", u8p), ("down", u8p),
        ("gate_f32", f32p), ("up_f32", f32p), ("down_f32", f32p),
    ]


_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        h = C.CDLL(str(LIB_PATH))
        sigs = {
            "or_block_layout": (C.c_int, [C.c_uint32, C.POINTER(sz), C.POINTER(sz)]),
            "or_byte_size": (C.c_int, [C.c_uint32, sz, C.POINTER(sz)]),
            "or_f16_to_f32": (C.c_float, [C.c_uint16]),
            "or_get_scale_min_k4": (None, [C.c_int, u8p, u8p, u8p]),
            "or_unpack_q3_k_scales": (None, [u8p, i8p]),
            "or_dequant_into": (C.c_int, [C.c_uint32, u8p, sz, f32p, sz]),
            "or_dequantize": (C.c_int, [C.c_uint32, u8p, sz, f32p, sz]),
            "or_quantize_activation": (None, [f32p, sz, i8p, f32p]),
            "or_block_sums": (None, [i8p, sz, sz, i32p]),
            "or_int8_dot": (C.c_float, [C.c_uint32, u8p, i8p, f32p, i32p]),
            "or_matvec": (C.c_int, [C.c_uint32, u8p, sz, sz, sz, f32p, f32p, C.c_int]),
            "or_matmul": (C.c_int, [C.c_uint32, u8p, sz, sz, sz, f32p, sz, f32p, C.c_int]),
            "or_dot": (C.c_float, [f32p, f32p, sz]),
            "or_simd_matmul": (None, [f32p, sz, sz, f32p, sz, f32p, C.c_int]),
            "or_softmax": (None, [f32p, sz]),
            "or_expf": (None, [f32p, sz, f32p]),
            "or_silu": (None, [f32p, sz]),
            "or_gate": (None, [C.c_int, f32p, C.c_int, C.c_int, u32p, f32p]),
            "or_feed_forward_batch": (C.c_int, [C.POINTER(MoeLayerC), f32p, C.c_int, f32p, u32p, f32p,
                                                f32p, C.c_int]),
            "or_seeded": (None, [C.c_uint64, sz, C.c_float, f32p]),
            "or_bound": (C.c_float, [sz]),
            "or_synthesize_expert": (None, [C.c_uint32, C.c_int, C.c_int, f32p, f32p, f32p]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(h, name)
            fn.restype, fn.argtypes = res, args
        _lib = h
    return _lib


def _f(a):
    return a.ctypes.data_as(f32p)


def _u8(a):
    return a.ctypes.data_as(u8p)


def block_layout(qtype):
    e, b = sz(), sz()
    if lib().or_block_layout(qtype, C.byref(e), C.byref(b)):
        return None
    return e.value, b.value


def byte_size(qtype, n):
    out = sz()
    if lib().or_byte_size(qtype, n, C.byref(out)):
        raise ValueError("bad type or length")
    return out.value


def f16_to_f32(h: int) -> float:
    return lib().or_f16_to_f32(h)


def dequantize(qtype, raw, n, checked=True):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    fn = lib().or_dequantize if checked else lib().or_dequant_into
    rc = fn(qtype, _u8(raw), raw.size, _f(out), n)
    if rc:
        raise ValueError(f"dequantize refused (rc={rc})")
    return out


def quantize_activation(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.size, dtype=np.int8)
    s = np.empty(x.size // 32, dtype=np.float32)
    lib().or_quantize_activation(_f(x), x.size, q.ctypes.data_as(i8p), _f(s))
    return q, s


def block_sums(q, width):
    q = np.ascontiguousarray(q, dtype=np.int8)
    out = np.empty(q.size // width, dtype=np.int32)
    lib().or_block_sums(q.ctypes.data_as(i8p), q.size, width, out.ctypes.data_as(i32p))
    return out


def matmul(qtype, w, rows, cols, xs, n, threads=1):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    xs = np.ascontiguousarray(xs, dtype=np.float32).reshape(-1)
    out = np.empty(n * rows, dtype=np.float32)
    rc = lib().or_matmul(qtype, _u8(w), w.size, rows, cols, _f(xs), n, _f(out), threads)
    if rc:
        raise ValueError(f"matmul refused (rc={rc})")
    return out


def matvec(qtype, w, rows, cols, x, threads=1):
    return matmul(qtype, w, rows, cols, x, 1, threads)


def simd_matmul(m, rows, cols, xs, n, threads=1):
    m = np.ascontiguousarray(m, dtype=np.float32)
    xs = np.ascontiguousarray(xs, dtype=np.float32).reshape(-1)
    out = np.empty(n * rows, dtype=np.float32)
    lib().or_simd_matmul(_f(m), rows, cols, _f(xs), n, _f(out), threads)
    return out


def dot(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return lib().or_dot(_f(a), _f(b), a.size)


def softmax(x):
    x = np.array(x, dtype=np.float32, copy=True)
    lib().or_softmax(_f(x), x.size)
    return x


def expf(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().or_expf(_f(x), x.size, _f(y))
    return y


def silu(x):
    x = np.array(x, dtype=np.float32, copy=True)
    lib().or_silu(_f(x), x.size)
    return x


def gate(kind, scores, k):
    s = np.array(scores, dtype=np.float32, copy=True)
    ids = np.empty(k, dtype=np.uint32)
    w = np.empty(k, dtype=np.float32)
    lib().or_gate(kind, _f(s), s.size, k, ids.ctypes.data_as(u32p), _f(w))
    return ids, w


def feed_forward_batch(layer: dict, hs, logits=None, threads=1):
    """layer: d, f, ne, k, gating, combine, packed, router, qtypes (g,u,d), gate, up, down
    (stacked uint8 arrays) and optionally gate_f32/up_f32/down_f32."""
    keep = []
    L = MoeLayerC()
    L.d, L.f, L.ne, L.k = layer["d"], layer["f"], layer["ne"], layer["k"]
    L.gating, L.combine, L.packed = layer.get("gating", 0), layer.get("combine", 0), layer.get("packed", 1)
    router = np.ascontiguousarray(layer["router"], dtype=np.float32)
    keep.append(router)
    L.router = _f(router)
    L.qt_gate, L.qt_up, L.qt_down = layer["qtypes"]
    for name in ("gate", "up", "down"):
        a = np.ascontiguousarray(layer[name], dtype=np.uint8)
        keep.append(a)
        setattr(L, name, _u8(a))
        fa = layer.get(name + "_f32")
        if fa is not None:
            fa = np.ascontiguousarray(fa, dtype=np.float32)
            keep.append(fa)
            setattr(L, name + "_f32", _f(fa))
    hs = np.ascontiguousarray(hs, dtype=np.float32)
    n = hs.shape[0]
    out = np.empty((n, L.d), dtype=np.float32)
    ids = np.empty((n, L.k), dtype=np.uint32)
    w = np.empty((n, L.k), dtype=np.float32)
    lp = None
    if logits is not None:
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        keep.append(logits)
        lp = _f(logits)
    rc = lib().or_feed_forward_batch(C.byref(L), _f(hs), n, _f(out), ids.ctypes.data_as(u32p), _f(w), lp, threads)
    if rc:
        raise ValueError(f"feed_forward_batch refused (rc={rc})")
    return out, ids, w


def seeded(seed, n, bound):
    out = np.empty(n, dtype=np.float32)
    lib().or_seeded(seed, n, bound, _f(out))
    return out


def synthesize_expert(eid, d=128, f=256):
    g = np.empty(f * d, dtype=np.float32)
    u = np.empty(f * d, dtype=np.float32)
    dn = np.empty(d * f, dtype=np.float32)
    lib().or_synthesize_expert(eid, d, f, _f(g), _f(u), _f(dn))
    return g, u, dn
