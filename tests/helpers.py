"""Test-data generators restated from the reference's own tests.

`splitmix64`, `half_bits`, `random_block` and `random_rows` follow
garuda/src/quant/mod.rs:1079-1178 (the helpers of its test module), so the tests
here feed the oracle and the GPU the same kind of inputs the reference's tests use,
with the same seeds.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

MASK = (1 << 64) - 1


class SplitMix:
    """quant/mod.rs:1097-1103"""

    def __init__(self, seed: int):
        self.s = seed & MASK

    def next(self) -> int:
        self.s = (self.s + 0x9E3779B97F4A7C15) & MASK
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
        return z ^ (z >> 31)


def half_bits(v: float) -> int:
    """quant/mod.rs:1079-1094: truncating f32 -> f16, normals only, tiny -> 0."""
    v = np.float32(v)
    if v == 0:
        return 0
    bits = int(np.array([v], dtype=np.float32).view(np.uint32)[0])
    sign = (bits >> 16) & 0x8000
    exp = ((bits >> 23) & 0xFF) - 127 + 15
    mant = bits & 0x7FFFFF
    if exp <= 0:
        return sign
    if exp >= 0x1F:
        return sign | 0x7C00
    return sign | (exp << 10) | (mant >> 13)


def random_block(qtype: int, rng: SplitMix) -> bytes:
    """quant/mod.rs:1134-1160"""
    _, nbytes = O.block_layout(qtype)
    b = bytearray(rng.next() % 256 for _ in range(nbytes))

    def small():
        return half_bits(np.float32(0.002) + np.float32(rng.next() % 100) * np.float32(0.0002))

    def tiny():
        return half_bits(np.float32(rng.next() % 40) * np.float32(0.0002))

    def put(off, h):
        b[off] = h & 0xFF
        b[off + 1] = h >> 8

    if qtype in (O.Q4_K, O.Q5_K):
        put(0, small())
        put(2, tiny())
    elif qtype == O.Q2_K:
        put(80, small())
        put(82, tiny())
    elif qtype == O.Q3_K:
        put(108, small())
    elif qtype == O.Q6_K:
        put(208, small())
    elif qtype == O.Q8_0:
        for blk in range(0, nbytes, 34):
            put(blk, small())
    else:
        raise ValueError(qtype)
    return bytes(b)


def random_rows(qtype: int, rows: int, cols: int, rng: SplitMix) -> np.ndarray:
    """quant/mod.rs:1163-1178"""
    n = O.byte_size(qtype, cols) * rows
    if qtype in O.INT8_TYPES:
        _, nb = O.block_layout(qtype)
        return np.frombuffer(b"".join(random_block(qtype, rng) for _ in range(n // nb)), dtype=np.uint8).copy()
    if qtype == O.F32:
        vals = [np.float32((rng.next() % 2000) / np.float32(1000.0)) - np.float32(1.0) for _ in range(n // 4)]
        return np.array(vals, dtype=np.float32).view(np.uint8).copy()
    return np.array([rng.next() % 64 for _ in range(n)], dtype=np.uint8)


def ref_x(rng: SplitMix, n: int, period: int) -> np.ndarray:
    """((splitmix % 2000) / 1000 - 1) * (1 + i % period), as the reference tests build x."""
    out = np.empty(n, dtype=np.float32)
    for i in range(n):
        v = np.float32(rng.next() % 2000) / np.float32(1000.0) - np.float32(1.0)
        out[i] = v * np.float32(1 + i % period)
    return out


def fast_random_blocks(qtype: int, nblocks: int, seed: int) -> np.ndarray:
    """Many valid blocks quickly (numpy): random bytes with plausible f16 scale fields,
    the same recipe as random_block but vectorised, for large parity tests."""
    e, nb = O.block_layout(qtype)
    r = np.random.default_rng(seed)
    b = r.integers(0, 256, size=(nblocks, nb), dtype=np.uint8)

    def halfs(lo, hi, size):
        return np.float16(r.uniform(lo, hi, size=size).astype(np.float32)).view(np.uint16)

    def put(off, h):
        b[:, off] = (h & 0xFF).astype(np.uint8)
        b[:, off + 1] = (h >> 8).astype(np.uint8)

    if qtype in (O.Q4_K, O.Q5_K):
        put(0, halfs(0.002, 0.022, nblocks))
        put(2, halfs(0.0, 0.008, nblocks))
    elif qtype == O.Q2_K:
        put(80, halfs(0.002, 0.022, nblocks))
        put(82, halfs(0.0, 0.008, nblocks))
    elif qtype == O.Q3_K:
        put(108, halfs(0.002, 0.022, nblocks))
    elif qtype == O.Q6_K:
        put(208, halfs(0.002, 0.022, nblocks))
    elif qtype in (O.Q8_0, O.Q4_0):
        put(0, halfs(0.002, 0.022, nblocks))
    elif qtype == O.F16:
        b = halfs(-1.0, 1.0, nblocks * e).view(np.uint8).reshape(nblocks, nb)
    elif qtype == O.F32:
        b = r.uniform(-1, 1, size=nblocks * e).astype(np.float32).view(np.uint8).reshape(nblocks, nb)
    return b.reshape(-1).copy()

