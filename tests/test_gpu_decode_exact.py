"""Decode-sized packed-math calls whose outputs are bit-exact against the oracle.

With a one-hot Q8_0 down matrix (one nonzero per row), each down row is one term
ws * xs * q * hq of one int8 code of h, and every other block adds an exact zero, so the
down product is the reference's (quant/mod.rs:398-407) bit for bit whatever order its
blocks are summed in; a top-2 combine of two terms is exact in any order too. The layer's
output is then bit-exact exactly when gate and up are: their integer sub-block dots and
the reference's float term per sub-block in K order (quant/mod.rs:417-621), and h's int8
requantisation (:331-345). One code of h rounded the other way changes an output.

The batches cover the v_dot4 path (chunks of one token) and the matrix-core path (chunks
of two or more: groups of four tokens, a partial last group), with Zipf-skewed routing so
that one expert takes most tokens. Every int8 gate/up type; routing bit-exact.
"""
import os

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import moe as M
from oracle import oracle as O
from tests.test_gpu_parity import bits, say
from tests.test_gpu_prefill_packed import onehot_down

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=1 << 30)
    yield d
    d.close()


@pytest.mark.parametrize("qt", [G.Q4_K, G.Q5_K, G.Q6_K, G.Q3_K, G.Q2_K, G.Q8_0])
def test_decode_gateup_is_bit_exact(dev, qt):
    d, f, ne, k = 512, 512, 8, 2
    rng = np.random.default_rng(90 + qt)
    gate = M.quantize(qt, rng.normal(0, 0.05, ne * f * d).astype(np.float32))
    up = M.quantize(qt, rng.normal(0, 0.05, ne * f * d).astype(np.float32))
    down = onehot_down(rng, ne, d, f)
    u = M.skew_direction(91 + qt, d)
    router = M.skew_router(rng.normal(0, 0.02, ne * d).astype(np.float32), ne, d, u)
    qts = (qt, qt, G.Q8_0)
    layer = G.MoeLayer(dev, d, f, ne, k, router, gate, up, down, qts, math=G.MATH_PACKED)
    L = dict(d=d, f=f, ne=ne, k=k, gating=0, combine=0, packed=1, router=router, qtypes=qts,
             gate=gate, up=up, down=down)
    try:
        for n in (1, 2, 3, 5, 8, 13):
            say(f"decode bit-exact, gate/up type {qt}, n={n}")
            hs = M.skew_tokens(rng.normal(0, 1, (n, d)).astype(np.float32), u)
            out, ids, w = layer.feed_forward_batch(hs)
            say(f"  expert loads: {np.bincount(ids.reshape(-1), minlength=ne).tolist()}")
            wout, wids, ww = O.feed_forward_batch(L, hs, threads=min(16, len(os.sched_getaffinity(0))))
            assert np.array_equal(ids, wids), "routing differs"
            assert np.array_equal(bits(w), bits(ww)), "routing weights differ"
            got = out.astype(np.float32)
            want = np.asarray(wout, dtype=np.float32)
            bad = np.flatnonzero(bits(got) != bits(want))
            assert bad.size == 0, (f"n={n}: {bad.size} outputs differ, first at {bad[0]}: "
                                   f"{got.reshape(-1)[bad[0]]!r} vs {want.reshape(-1)[bad[0]]!r}")
    finally:
        layer.release()


@pytest.mark.parametrize("qt", [G.Q4_K, G.Q5_K, G.Q6_K, G.Q3_K, G.Q2_K])
@pytest.mark.parametrize("d", [2048, 1280])
def test_split_gateup_is_bit_exact(dev, qt, d):
    """Single-token calls with four or more units a row run the gate/up tile's K range
    split over four waves a matrix (k_gu_split: terms kept, then added in K order); the
    outputs stay bit-exact, also with parts of unequal length (d 1280: 5 units), and the
    two-token calls between them (k_gu_units) too."""
    f, ne, k = 512, 8, 2
    rng = np.random.default_rng(190 + qt + d)
    gate = M.quantize(qt, rng.normal(0, 0.05, ne * f * d).astype(np.float32))
    up = M.quantize(qt, rng.normal(0, 0.05, ne * f * d).astype(np.float32))
    down = onehot_down(rng, ne, d, f)
    u = M.skew_direction(191 + qt, d)
    router = M.skew_router(rng.normal(0, 0.02, ne * d).astype(np.float32), ne, d, u)
    qts = (qt, qt, G.Q8_0)
    layer = G.MoeLayer(dev, d, f, ne, k, router, gate, up, down, qts, math=G.MATH_PACKED)
    L = dict(d=d, f=f, ne=ne, k=k, gating=0, combine=0, packed=1, router=router, qtypes=qts,
             gate=gate, up=up, down=down)
    try:
        for n in (1, 2, 1, 2):
            say(f"split gate/up bit-exact, type {qt}, d={d}, n={n}")
            hs = M.skew_tokens(rng.normal(0, 1, (n, d)).astype(np.float32), u)
            out, ids, w = layer.feed_forward_batch(hs)
            wout, wids, ww = O.feed_forward_batch(L, hs, threads=min(16, len(os.sched_getaffinity(0))))
            assert np.array_equal(ids, wids), "routing differs"
            assert np.array_equal(bits(w), bits(ww)), "routing weights differ"
            got = out.astype(np.float32)
            want = np.asarray(wout, dtype=np.float32)
            bad = np.flatnonzero(bits(got) != bits(want))
            assert bad.size == 0, (f"n={n}: {bad.size} outputs differ, first at {bad[0]}: "
                                   f"{got.reshape(-1)[bad[0]]!r} vs {want.reshape(-1)[bad[0]]!r}")
    finally:
        layer.release()


@pytest.mark.parametrize("f", [768, 1280])
def test_single_token_down_in_half_tiles(dev, f):
    """One token's down product runs in half tiles whose half-waves stream alternate units
    (k_dn_atomic's PAIR form); with 3 or 5 units a row (f 768, 1280) the last pair has one
    unit. The one-hot down keeps the output bit-exact whatever the summation order, so
    every row of every half tile must be the reference's."""
    d, ne, k, qt = 512, 8, 2, G.Q4_K
    rng = np.random.default_rng(290 + f)
    gate = M.quantize(qt, rng.normal(0, 0.05, ne * f * d).astype(np.float32))
    up = M.quantize(qt, rng.normal(0, 0.05, ne * f * d).astype(np.float32))
    down = onehot_down(rng, ne, d, f)
    u = M.skew_direction(291 + f, d)
    router = M.skew_router(rng.normal(0, 0.02, ne * d).astype(np.float32), ne, d, u)
    qts = (qt, qt, G.Q8_0)
    layer = G.MoeLayer(dev, d, f, ne, k, router, gate, up, down, qts, math=G.MATH_PACKED)
    L = dict(d=d, f=f, ne=ne, k=k, gating=0, combine=0, packed=1, router=router, qtypes=qts,
             gate=gate, up=up, down=down)
    try:
        for n in (1, 2, 1):
            say(f"half-tile down, f={f}, n={n}")
            hs = M.skew_tokens(rng.normal(0, 1, (n, d)).astype(np.float32), u)
            out, ids, w = layer.feed_forward_batch(hs)
            wout, wids, ww = O.feed_forward_batch(L, hs, threads=min(16, len(os.sched_getaffinity(0))))
            assert np.array_equal(ids, wids), "routing differs"
            got = out.astype(np.float32)
            want = np.asarray(wout, dtype=np.float32)
            bad = np.flatnonzero(bits(got) != bits(want))
            assert bad.size == 0, (f"n={n}: {bad.size} outputs differ, first at {bad[0]}: "
                                   f"{got.reshape(-1)[bad[0]]!r} vs {want.reshape(-1)[bad[0]]!r}")
    finally:
        layer.release()
