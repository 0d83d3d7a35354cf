"""Routing on non-finite router inputs, on the GPU, through every front end, against the
oracle: ids and weights bit for bit, under all four gatings.

The reference defines most of these cases. simd::softmax falls back to uniform
probabilities when the maximum or the sum is not finite (simd/mod.rs:132-158), so llama,
DeepSeek and Qwen gating rank equal probabilities by id (llama/mod.rs:942-949,
router/mod.rs:84-88). Mixtral ranks the raw logits with partial_cmp, which is no order
once a logit is NaN (router/mod.rs:83-88: Rust's sort_by then gives an unspecified order
or panics). This build ranks a NaN after every number, NaNs among themselves by id, on the
device and in the oracle alike. That case is parity unpinned: nothing in the reference
fixes it. The softmax over the kept logits (router/mod.rs:91-97) is uniform when one of
them is NaN or infinite.

Front ends: k_spec_front (decode, logits computed here: NaN and +-inf reach the logits
through the activations, or through one activation times a large router weight, which
overflows to +-inf for chosen experts only), k_front (given logits; or more tokens than
the speculative front end takes), k_front_wide (64 < experts <= 256) and k_route (more
experts, or experts not resident). Outputs of the tokens whose inputs are all finite are
checked against the oracle within the layer bar: a token with a NaN never disturbs
another.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import garuda_amd as G
from oracle import oracle as O
from tests.test_gpu_parity import ATOL, RTOL, bits, make_layer, oracle_layer, say

pytestmark = pytest.mark.gpu
GATINGS = (G.GATING_LLAMA, G.GATING_MIXTRAL, G.GATING_DEEPSEEK, G.GATING_QWEN)
THREADS = min(16, len(os.sched_getaffinity(0)))


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=1 << 30)
    yield d
    d.close()


def bad_logits(rng, n, ne):
    """Given logits: token 0 finite, token 1 a NaN, token 2 +inf, token 3 -inf beside
    finite values, token 4 all NaN, token 5 NaN and +-inf mixed with ties; the rest a mix."""
    x = rng.normal(0, 2, (n, ne)).astype(np.float32)
    rows = [[], [(1, np.nan)], [(2, np.inf)], [(0, -np.inf), (3, -np.inf)], None,
            [(0, np.nan), (1, np.inf), (2, -np.inf), (4, np.nan)]]
    for t in range(1, n):
        spec = rows[t] if t < len(rows) else [(int(j), [np.nan, np.inf, -np.inf][t % 3])
                                             for j in rng.choice(ne, size=min(ne, 1 + t % 4), replace=False)]
        if spec is None:
            x[t] = np.nan
            continue
        for j, v in spec:
            x[t, j % ne] = v
        if t == 5:
            x[t, 5 % ne] = x[t, 6 % ne]  # a tie among the numbers
    return x


def compare(layer, L, hs, logits, finite_rows):
    out, ids, w = layer.feed_forward_batch(hs, logits)
    wout, wids, ww = O.feed_forward_batch(L, hs, logits, threads=THREADS)
    assert np.array_equal(ids, wids), f"routing differs:\n{ids}\n{wids}"
    assert np.array_equal(bits(w), bits(ww)), f"routing weights differ:\n{w}\n{ww}"
    assert ids.max() < L["ne"]
    if finite_rows:
        r = list(finite_rows)
        assert np.allclose(out[r], wout[r], rtol=RTOL, atol=ATOL), np.abs(out[r] - wout[r]).max()


def layer_pair(dev, seed, d, f, ne, k, gating, qts=(G.Q4_K,) * 3, router_fn=None):
    rng = np.random.default_rng(seed)
    router, mats = make_layer(rng, d, f, ne, qts[0], qts[2])
    if router_fn is not None:
        router = np.ascontiguousarray(router_fn(router.reshape(ne, d).copy()).astype(np.float32).reshape(-1))
    layer = G.MoeLayer(dev, d, f, ne, k, router, mats["gate"], mats["up"], mats["down"], qts, gating=gating,
                       math=G.MATH_PACKED)
    return rng, layer, oracle_layer(d, f, ne, k, router, mats, qts, G.MATH_PACKED, gating)


@pytest.mark.parametrize("gating", GATINGS)
def test_given_logits_k_front(dev, gating):
    # ne <= 64 with logits given: k_front (and its dispatch), at a decode and a larger batch
    rng, layer, L = layer_pair(dev, 300 + gating, 256, 512, 8, 2, gating)
    try:
        for n in (6, 9, 70):
            say(f"k_front non-finite logits, gating {gating}, n={n}")
            hs = rng.normal(0, 1, (n, 256)).astype(np.float32)
            compare(layer, L, hs, bad_logits(rng, n, 8), [0])
    finally:
        layer.release()


@pytest.mark.parametrize("gating", GATINGS)
def test_computed_logits_speculative_and_k_front(dev, gating):
    """Logits computed on the device from non-finite activations: k_spec_front at decode
    batches (its rigorous bound makes every expert a candidate of a non-finite token, and
    the exact routing chain picks), k_front at 80 tokens. Column 0 of the router is +40 for
    expert 2, -40 for expert 5 and 0 elsewhere: an activation of 1e37 there makes those two
    logits +inf and -inf and leaves the others finite."""
    def router_fn(r):
        r[:, 0] = 0.0
        r[2, 0], r[5, 0] = 40.0, -40.0
        return r

    rng, layer, L = layer_pair(dev, 310 + gating, 256, 512, 8, 2, gating, router_fn=router_fn)
    try:
        for n in (1, 4, 8, 80):
            say(f"computed non-finite logits, gating {gating}, n={n}")
            hs = rng.normal(0, 1, (n, 256)).astype(np.float32)
            finite = []
            for t in range(n):
                kind = t % 5
                if kind == 1:
                    hs[t, 7] = np.nan
                elif kind == 2:
                    hs[t, 0] = 1e37  # expert 2 +inf, expert 5 -inf
                elif kind == 3:
                    hs[t, 9] = np.inf  # +-inf or NaN in every logit
                elif kind == 4:
                    hs[t, 0] = -1e37  # expert 2 -inf, expert 5 +inf
                else:
                    finite.append(t)
            if n == 1:
                hs[0, 0] = 1e37
                finite = []
            compare(layer, L, hs, None, finite)
    finally:
        layer.release()


@pytest.mark.parametrize("gating", GATINGS)
def test_wide_front_end(dev, gating):
    # 128 experts, top-8: k_front_wide, logits given and computed
    rng, layer, L = layer_pair(dev, 320 + gating, 256, 256, 128, 8, gating, qts=(G.Q6_K, G.Q6_K, G.Q8_0))
    try:
        for n in (6, 40):
            say(f"k_front_wide non-finite, gating {gating}, n={n}")
            hs = rng.normal(0, 1, (n, 256)).astype(np.float32)
            compare(layer, L, hs, bad_logits(rng, n, 128), [0])
            hs2 = hs.copy()
            hs2[1::3, 11] = np.nan
            hs2[2::3, 13] = np.inf
            compare(layer, L, hs2, None, [t for t in range(n) if t % 3 == 0])
    finally:
        layer.release()


@pytest.mark.parametrize("gating", GATINGS)
def test_route_front_end_many_experts(dev, gating):
    # 300 experts (past k_front_wide's 256): k_route's per-thread gating (gate_block)
    rng, layer, L = layer_pair(dev, 330 + gating, 128, 128, 300, 4, gating, qts=(G.Q8_0,) * 3)
    try:
        n = 12
        say(f"k_route non-finite, gating {gating}")
        hs = rng.normal(0, 1, (n, 128)).astype(np.float32)
        compare(layer, L, hs, bad_logits(rng, n, 300), [0])
    finally:
        layer.release()


def test_route_front_end_experts_not_resident():
    # a slab of two experts: a forward whose experts are not all resident routes exactly
    # first (k_route) and stages what it routed; non-finite logits must not route outside
    # the layer or stage a wrong expert
    d, f, ne, k = 256, 256, 8, 2
    for gating in GATINGS:
        rng = np.random.default_rng(340 + gating)
        router, mats = make_layer(rng, d, f, ne, G.Q4_K, G.Q4_K)
        per = 3 * O.byte_size(G.Q4_K, f * d)
        with G.Device(0, slab_bytes=2 * per + (1 << 16)) as small:
            layer = G.MoeLayer(small, d, f, ne, k, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3,
                               gating=gating, math=G.MATH_PACKED)
            L = oracle_layer(d, f, ne, k, router, mats, (G.Q4_K,) * 3, G.MATH_PACKED, gating)
            try:
                for t in range(4):
                    say(f"not resident, gating {gating}, call {t}")
                    hs = rng.normal(0, 1, (1, d)).astype(np.float32)
                    if t % 2:
                        hs[0, 3] = [np.nan, np.inf][t // 2]
                    compare(layer, L, hs, None, [] if t % 2 else [0])
            finally:
                layer.release()
