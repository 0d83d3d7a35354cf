"""Decode attention over a paged KV cache on the device: the reference's
`LlamaBackend::attend_one` (garuda/src/llama/mod.rs:766-821) over per-sequence,
per-layer `KVCacheState`s (garuda/src/cache/mod.rs:221-600), backed by gmoe_kv_* and
gmoe_attention* (include/garuda_moe.h).

`KvCache.attention(layer, seqs, q, k, v)` takes one token per entry, rotates q and k
by the token's position (simd::rope), appends k and v to that sequence's cache for the
layer, and returns each token's attention context. Several entries of one sequence are
its consecutive positions, so a prompt can be prefilled in one call.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import lib
from .moe import _check, _fp


class GmoeKvDesc(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("block_size", C.c_uint32), ("max_positions", C.c_uint32),
                ("sliding_window", C.c_uint32), ("max_seqs", C.c_uint32), ("max_pages", C.c_uint64),
                ("rope_theta", C.c_float)]


class KvCache:
    def __init__(self, dev, n_layers: int, n_heads: int, n_kv_heads: int, head_dim: int, block_size: int = 16,
                 max_positions: int = 2048, sliding_window: int = 0, max_seqs: int = 8, max_pages: int | None = None,
                 rope_theta: float = 10000.0):
        if max_pages is None:
            max_pages = max_seqs * n_layers * ((max_positions + block_size - 1) // block_size)
        self.dev = dev
        self.n_layers, self.n_heads, self.n_kv, self.hd = n_layers, n_heads, n_kv_heads, head_dim
        self.kv_dim = n_kv_heads * head_dim
        d = GmoeKvDesc(n_layers, n_heads, n_kv_heads, head_dim, block_size, max_positions, sliding_window, max_seqs,
                       max_pages, rope_theta)
        h = C.c_void_p()
        _check(lib().gmoe_kv_create(dev.handle, C.byref(d), C.byref(h)))
        self._h = h

    def open_seq(self) -> int:
        s = C.c_uint32()
        _check(lib().gmoe_kv_seq_open(self._h, C.byref(s)))
        return s.value

    def close_seq(self, seq: int) -> None:
        _check(lib().gmoe_kv_seq_close(self._h, seq))

    def seq_len(self, seq: int, layer: int = 0) -> int:
        n = C.c_uint32()
        _check(lib().gmoe_kv_seq_len(self._h, seq, layer, C.byref(n)))
        return n.value

    def free_pages(self) -> int:
        n = C.c_uint64()
        _check(lib().gmoe_kv_free_pages(self._h, C.byref(n)))
        return n.value

    def fail_reserves(self, count: int) -> None:
        """Test hook: the next `count` attention-scratch reservations of graph-replayed
        model steps fail as a device allocation would."""
        _check(lib().gmoe_kv_fail_reserves(self._h, count))

    def attention(self, layer: int, seqs, q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
        seqs = np.ascontiguousarray(np.asarray(seqs, dtype=np.uint32).reshape(-1))
        n = seqs.size
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(n, self.n_heads * self.hd)
        k = np.ascontiguousarray(k, dtype=np.float32).reshape(n, self.kv_dim)
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(n, self.kv_dim)
        out = np.empty((n, self.n_heads * self.hd), dtype=np.float32)
        _check(lib().gmoe_attention(self._h, layer, seqs.ctypes.data_as(C.POINTER(C.c_uint32)), n, _fp(q), _fp(k),
                                    _fp(v), _fp(out)))
        return out

    def attention_async(self, layer: int, seqs, d_q: int, d_k: int, d_v: int, d_out: int, stream: int = 0) -> None:
        seqs = np.ascontiguousarray(np.asarray(seqs, dtype=np.uint32).reshape(-1))
        _check(lib().gmoe_attention_async(self._h, layer, seqs.ctypes.data_as(C.POINTER(C.c_uint32)), seqs.size,
                                          d_q or None, d_k or None, d_v or None, d_out or None, stream or None))

    def close(self) -> None:
        if self._h is not None:
            lib().gmoe_kv_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()
