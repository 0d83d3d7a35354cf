"""Packed-math prefill on MFMA (k_pq) through the C-ABI, against the oracle.

Prefill-sized calls under packed math (Weight::Packed, mmap = true) run quant::matmul's
int8 arithmetic (quant/mod.rs:223-304, :398-621) with the sub-block dots on fp16 MFMAs.
Two bars:

* gate/up's int8 codes exactly: with a one-hot Q8_0 down matrix every down row has one
  nonzero term, w * scale * q of one h value. The down product runs on the dequantised h
  split into two fp16 halves (22 significant bits), so each term is the reference's
  within about 2^-22 of itself, while one int8 code of h rounded the other way would move
  it by at least 1/127 of itself. An error bound of 2e-6 of the outputs' size therefore
  pins every code (and every scale to a few ulps): the MFMA dots and the K-ordered float
  chain of every int8 gate/up type.
* the whole layer within rtol 1e-3 / atol 1e-4 (the down product splits K into slices
  that the combine adds in order), for down types with and without sums.

Token loads are Zipf(1.1)-skewed, so experts get ragged token counts: tiles of 64 with
a partial last one, experts below one 8-token group, and idle experts.
"""
import os

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import moe as M
from oracle import oracle as O
from tests.test_gpu_parity import ATOL, RTOL, bits, check_layer, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=3 << 30)
    yield d
    d.close()


def onehot_down(rng, ne, d, f):
    """Q8_0 down matrices [ne][d][f] with one nonzero per row."""
    x = np.zeros((ne, d, f), np.float32)
    cols = rng.integers(0, f, (ne, d))
    vals = rng.normal(0, 0.05, (ne, d)).astype(np.float32)
    for e in range(ne):
        x[e, np.arange(d), cols[e]] = vals[e]
    return M.quantize(G.Q8_0, x.reshape(-1))


@pytest.mark.parametrize("qt", [G.Q4_K, G.Q5_K, G.Q6_K, G.Q3_K, G.Q2_K, G.Q8_0])
def test_packed_prefill_gateup_codes_are_exact(dev, qt):
    d, f, ne, k = 512, 512, 8, 2
    rng = np.random.default_rng(60 + qt)
    gate = M.quantize(qt, rng.normal(0, 0.05, ne * f * d).astype(np.float32))
    up = M.quantize(qt, rng.normal(0, 0.05, ne * f * d).astype(np.float32))
    down = onehot_down(rng, ne, d, f)
    router = rng.normal(0, 0.02, ne * d).astype(np.float32)
    u = M.skew_direction(61 + qt, d)
    router = M.skew_router(router, ne, d, u)
    qts = (qt, qt, G.Q8_0)
    layer = G.MoeLayer(dev, d, f, ne, k, router, gate, up, down, qts, math=G.MATH_PACKED)
    L = dict(d=d, f=f, ne=ne, k=k, gating=0, combine=0, packed=1, router=router, qtypes=qts,
             gate=gate, up=up, down=down)
    try:
        for n in (64, 300):
            say(f"packed prefill gate/up type {qt}, n={n}")
            hs = M.skew_tokens(rng.normal(0, 1, (n, d)).astype(np.float32), u)
            out, ids, w = layer.feed_forward_batch(hs)
            say(f"  expert loads: {np.bincount(ids.reshape(-1), minlength=ne).tolist()}")
            wout, wids, ww = O.feed_forward_batch(L, hs, threads=min(16, len(os.sched_getaffinity(0))))
            assert np.array_equal(ids, wids), "routing differs"
            assert np.array_equal(bits(w), bits(ww)), "routing weights differ"
            err = np.abs(out.astype(np.float64) - wout)
            bound = 2e-6 * (np.abs(wout) + np.abs(wout).max())
            bad = np.flatnonzero(err > bound)
            assert bad.size == 0, (f"{bad.size} outputs beyond 2e-6, first at {bad[0]}: "
                                   f"{out.reshape(-1)[bad[0]]} vs {wout.reshape(-1)[bad[0]]}")
    finally:
        layer.release()


@pytest.mark.parametrize("qts", [(G.Q4_K,) * 3, (G.Q5_K,) * 3, (G.Q6_K,) * 3, (G.Q3_K, G.Q3_K, G.Q4_K),
                                 (G.Q2_K,) * 3, (G.Q8_0,) * 3, (G.Q6_K, G.Q6_K, G.Q8_0)])
def test_packed_prefill_every_type(dev, qts):
    worst = check_layer(dev, 512, 1024, 8, 2, qts, (64, 300), G.MATH_PACKED, seed=70 + qts[0] + qts[2], zipf=True)
    # h is exact, so the only differences are the down product's reordered f32 sums
    assert worst < 0.05, f"worst error {worst:.3g} of the tolerance: more than reordered sums give"


def test_packed_prefill_many_tiles(dev):
    # d 1024, f 2048, 512 Zipf tokens: the busiest expert spans several 64-token tiles
    check_layer(dev, 1024, 2048, 8, 2, (G.Q4_K,) * 3, (512,), G.MATH_PACKED, seed=80, zipf=True)


def test_packed_prefill_at_the_threshold(dev):
    # 64 tokens of top-2 over 8 experts are 128 pairs: the smallest call k_pq takes,
    # next to 63 tokens, which the decode kernels take
    check_layer(dev, 512, 512, 8, 2, (G.Q4_K,) * 3, (63, 64), G.MATH_PACKED, seed=81)
