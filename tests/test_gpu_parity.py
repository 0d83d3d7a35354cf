"""GPU parity: every step of the path through the C-ABI against the oracle.

Bars: routing indices, expert assignment, dequantised
weights and exp bit-exact; layer outputs within rtol 1e-3 / atol 1e-4 in fp32 of the
reference path with the same arithmetic (PACKED <-> Weight::Packed / mmap = true,
F32 <-> Weight::Full / mmap = false).
"""
import os
import sys

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import moe as M
from oracle import oracle as O
from tests.helpers import fast_random_blocks

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=3 << 30)
    yield d
    d.close()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---------------- exp ----------------

def test_device_expf_is_bit_exact_to_host_libm(dev):
    say("expf sweep")
    u = np.arange(0, 1 << 32, 61, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    x = x[(x > -110) & (x < 95)]
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 88.72283, 88.72284, -103.97208, -103.97209,
                        -87.33655, 1e-30, -1e-30], np.float32)
    x = np.concatenate([x, special]).astype(np.float32)
    got = dev.expf(x)
    want = O.expf(x)
    same = (bits(got) == bits(want)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), f"{(~same).sum()} of {x.size} differ, first x={x[~same][:4]}"


# ---------------- dequant ----------------

@pytest.mark.parametrize("qtype", [G.Q4_K, G.Q5_K, G.Q6_K, G.Q3_K, G.Q2_K, G.Q8_0, G.Q4_0, G.F16, G.F32])
def test_dequant_is_bit_exact(dev, qtype):
    e, _ = O.block_layout(qtype)
    nblk = 4096 if e > 1 else 4096 * 32
    raw = fast_random_blocks(qtype, nblk, 100 + qtype)
    n = nblk * e
    got = dev.dequantize(qtype, raw, n)
    want = O.dequantize(qtype, raw, n, checked=False)
    same = (bits(got) == bits(want)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


# ---------------- single matrix products ----------------

@pytest.mark.parametrize("math", [G.MATH_PACKED, G.MATH_F32])
@pytest.mark.parametrize("qtype", [G.Q4_K, G.Q5_K, G.Q6_K, G.Q3_K, G.Q2_K, G.Q8_0, G.Q4_0, G.F16, G.F32])
def test_matmul_matches_reference_path(dev, qtype, math):
    e, _ = O.block_layout(qtype)
    rows, cols = 67, (1024 if e == 256 else 256)
    for n in (1, 3, 8):
        raw = fast_random_blocks(qtype, rows * cols // e, 7 + qtype + n)
        xs = np.random.default_rng(n).normal(0, 1, n * cols).astype(np.float32)
        got = dev.matmul(qtype, raw, rows, cols, xs, n, math)
        deq = O.dequantize(qtype, raw, rows * cols, checked=False).reshape(rows, cols)
        if math == G.MATH_PACKED:
            want = O.matmul(qtype, raw, rows, cols, xs, n)
        else:
            want = O.simd_matmul(deq, rows, cols, xs, n)
        # summation order is the only difference: bound it by the magnitude of the terms
        scale = (np.abs(deq)[None] * np.abs(xs.reshape(n, 1, cols))).sum(-1).reshape(-1)
        assert (np.abs(got - want) <= 1e-5 * scale + 1e-6).all(), f"n={n}"


# ---------------- routing and dispatch ----------------

@pytest.mark.parametrize("gating", [G.GATING_LLAMA, G.GATING_MIXTRAL, G.GATING_DEEPSEEK, G.GATING_QWEN])
@pytest.mark.parametrize("ne,k,d", [(8, 2, 4096), (128, 8, 2048), (4, 2, 32), (64, 6, 256)])
def test_route_is_bit_exact(dev, gating, ne, k, d):
    rng = np.random.default_rng(ne * 7 + k + gating)
    n = 37
    router = rng.normal(0, 0.02, (ne, d)).astype(np.float32)
    hs = rng.normal(0, 1, (n, d)).astype(np.float32)
    hs[5] = hs[4]  # identical tokens route identically
    ids, w, logits = dev.route(gating, router, hs, ne, k)
    for t in range(n):
        want_l = O.simd_matmul(router, ne, d, hs[t], 1)
        assert np.array_equal(bits(logits[t]), bits(want_l)), f"logits t={t}"
        wi, ww = O.gate(gating, want_l, k)
        assert (ids[t] == wi).all(), f"ids t={t}"
        assert np.array_equal(bits(w[t]), bits(ww)), f"weights t={t}"


@pytest.mark.parametrize("gating", [G.GATING_LLAMA, G.GATING_MIXTRAL])
def test_route_from_logits_with_ties(dev, gating):
    rng = np.random.default_rng(5)
    n, ne, k = 64, 128, 8
    logits = (rng.random((n, ne), dtype=np.float32) * np.float32(4)).astype(np.float32)
    logits[::3, 10:20] = logits[::3, 30:31]  # exact ties: lower id first
    logits[1] = 0.0
    ids, w, _ = dev.route(gating, None, logits, ne, k)
    for t in range(n):
        wi, ww = O.gate(gating, logits[t], k)
        assert (ids[t] == wi).all() and np.array_equal(bits(w[t]), bits(ww))


def test_dispatch_is_a_stable_counting_sort(dev):
    rng = np.random.default_rng(9)
    for n, k, ne in ((1, 2, 8), (8, 2, 8), (512, 2, 8), (64, 8, 128), (33, 3, 5)):
        ids = np.stack([rng.permutation(ne)[:k] for _ in range(n)]).astype(np.uint32)
        w = rng.random((n, k)).astype(np.float32)
        off, tok, sw, rank = dev.dispatch(ids, w, ne)
        flat = ids.reshape(-1)
        order = np.argsort(flat, kind="stable")
        assert np.array_equal(tok, (order // k).astype(np.uint32))
        assert np.array_equal(rank, (order % k).astype(np.uint32))
        assert np.array_equal(bits(sw), bits(w.reshape(-1)[order]))
        assert np.array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=ne))]).astype(np.uint32))


# ---------------- whole layers ----------------

def make_layer(rng, d, f, ne, qt_gu, qt_dn, wstd=0.02):
    mats = {}
    for name, rows, cols, qt in (("gate", f, d, qt_gu), ("up", f, d, qt_gu), ("down", d, f, qt_dn)):
        if ne * rows * cols > (1 << 26):  # full-size layers: the library's threaded generator
            x = M.fill_gaussian(int(rng.integers(1 << 62)), ne * rows * cols, 0.0, wstd, 16)
        else:
            x = rng.normal(0, wstd, ne * rows * cols).astype(np.float32)
        mats[name] = M.quantize(qt, x, 16)
    router = rng.normal(0, wstd, ne * d).astype(np.float32)
    return router, mats


def oracle_layer(d, f, ne, k, router, mats, qts, math, gating=0, combine=0):
    return dict(d=d, f=f, ne=ne, k=k, gating=gating, combine=combine, packed=1 if math == G.MATH_PACKED else 0,
                router=router, qtypes=qts, **mats)


def check_layer(dev, d, f, ne, k, qts, ns, math, gating=0, combine=0, seed=0, logits_scale=None, split=False,
                tie_logits=False, zipf=False, sample=None, router_fn=None):
    """zipf: tokens and router biased along one shared direction so the expert load
    follows Zipf(1.1); sample: compare only this many tokens (spread over the batch)
    with the oracle, which then runs on those tokens alone."""
    rng = np.random.default_rng(seed)
    router, mats = make_layer(rng, d, f, ne, qts[0], qts[2])
    if zipf:
        u = M.skew_direction(seed + 1, d)
        router = M.skew_router(router, ne, d, u)
    if router_fn is not None:
        router = np.ascontiguousarray(router_fn(router.reshape(ne, d).copy()).astype(np.float32).reshape(-1))
    gpu_mats = dict(mats)
    if split:
        for name, rows, cols in (("gate", f, d), ("up", f, d), ("down", d, f)):
            per = mats[name].size // ne
            gpu_mats[name] = [mats[name][e * per:(e + 1) * per] for e in range(ne)]
    layer = G.MoeLayer(dev, d, f, ne, k, router, gpu_mats["gate"], gpu_mats["up"], gpu_mats["down"], qts,
                       gating=gating, combine=combine, math=math)
    L = oracle_layer(d, f, ne, k, router, mats, qts, math, gating, combine)
    worst = 0.0
    try:
        for n in ns:
            say(f"layer d={d} f={f} ne={ne} k={k} qts={qts} math={math} gating={gating} n={n}")
            hs = rng.normal(0, 1, (n, d)).astype(np.float32)
            logits = None
            if logits_scale is not None:
                logits = (rng.random((n, ne), dtype=np.float32) * np.float32(logits_scale)).astype(np.float32)
            if tie_logits:  # four distinct values: most tokens have ties inside and across the top k
                logits = (rng.integers(0, 4, (n, ne)) * 0.5).astype(np.float32)
            if zipf:
                hs = M.skew_tokens(hs, u)
            out, ids, w = layer.feed_forward_batch(hs, logits)
            if zipf:
                say(f"  expert loads: {np.bincount(ids.reshape(-1), minlength=ne).tolist()}")
            if sample is not None and sample < n:
                pick = np.linspace(0, n - 1, sample).astype(np.int64)
                hs, out, ids, w = hs[pick], out[pick], ids[pick], w[pick]
                logits = None if logits is None else logits[pick]
            wout, wids, ww = O.feed_forward_batch(L, hs, logits, threads=min(16, len(os.sched_getaffinity(0))))
            assert np.array_equal(ids, wids), "routing differs"
            assert np.array_equal(bits(w), bits(ww)), "routing weights differ"
            err = np.abs(out - wout)
            worst = max(worst, float((err / (ATOL + RTOL * np.abs(wout))).max()))
            assert np.allclose(out, wout, rtol=RTOL, atol=ATOL), f"n={n} max err {err.max()}"
    finally:
        layer.release()
    say(f"  worst error as a fraction of the tolerance: {worst:.3g}")
    return worst


@pytest.mark.parametrize("math", [G.MATH_PACKED, G.MATH_F32])
def test_q4k_layer(dev, math):
    check_layer(dev, 256, 512, 8, 2, (G.Q4_K,) * 3, (1, 2, 5, 8, 64), math)


@pytest.mark.parametrize("qts", [(G.Q5_K,) * 3, (G.Q6_K,) * 3, (G.Q3_K, G.Q3_K, G.Q4_K), (G.Q2_K,) * 3,
                                 (G.Q8_0,) * 3, (G.Q6_K, G.Q6_K, G.Q8_0), (G.Q4_0,) * 3, (G.F16,) * 3,
                                 (G.F32,) * 3])
@pytest.mark.parametrize("math", [G.MATH_PACKED, G.MATH_F32])
def test_layer_every_type(dev, qts, math):
    check_layer(dev, 256, 512, 8, 2, qts, (1, 7, 20), math, seed=qts[0])


@pytest.mark.parametrize("gating,combine", [(1, 1), (2, 1), (3, 1), (0, 1), (1, 0)])
def test_layer_gating_variants(dev, gating, combine):
    check_layer(dev, 256, 512, 8, 2, (G.Q4_K,) * 3, (1, 9), G.MATH_PACKED, gating, combine, seed=gating)


@pytest.mark.parametrize("qts", [(G.Q4_K,) * 3, (G.Q6_K, G.Q6_K, G.Q8_0), (G.Q3_K, G.Q3_K, G.Q4_K), (G.Q8_0,) * 3])
@pytest.mark.parametrize("math", [G.MATH_PACKED, G.MATH_F32])
def test_wide_rows_split_over_waves(dev, qts, math):
    # d_model 4096 gives 16 units a row: decode batches of 1-2 tokens split each
    # gate/up row over 2-4 waves, larger ones keep one wave per row
    check_layer(dev, 4096, 512, 8, 2, qts, (1, 2, 3, 8), math, seed=6)


@pytest.mark.parametrize("gating", [G.GATING_LLAMA, G.GATING_MIXTRAL, G.GATING_DEEPSEEK, G.GATING_QWEN])
def test_front_end_given_logits_with_ties(dev, gating):
    # ties go to the lower expert id; one workgroup per token, the last one dispatching
    check_layer(dev, 256, 512, 8, 2, (G.Q4_K,) * 3, (1, 3, 8, 40), G.MATH_PACKED, gating, seed=7, tie_logits=True)


def test_front_end_64_experts(dev):
    check_layer(dev, 256, 256, 64, 6, (G.Q4_K,) * 3, (1, 5, 12), G.MATH_PACKED, seed=8)


# f32 math from kPfMinSlots = 64 slots runs the expert products on MFMA (exact fp16
# products, f32 sums) over token tiles of 64; Zipf-skewed loads give the busiest expert several
# tiles, the last one partial.
@pytest.mark.parametrize("qts", [(G.Q4_K,) * 3, (G.Q5_K,) * 3, (G.Q6_K,) * 3, (G.Q3_K, G.Q3_K, G.Q4_K),
                                 (G.Q2_K,) * 3, (G.Q8_0,) * 3, (G.Q6_K, G.Q6_K, G.Q8_0), (G.Q4_0,) * 3,
                                 (G.F16,) * 3])
def test_prefill_every_type(dev, qts):
    check_layer(dev, 256, 512, 8, 2, qts, (32, 300), G.MATH_F32, seed=20 + qts[0], zipf=True)


@pytest.mark.parametrize("qts", [(G.Q4_K,) * 3, (G.Q6_K, G.Q6_K, G.Q8_0), (G.Q4_0,) * 3])
def test_prefill_zipf_512_tokens(dev, qts):
    # 1024 slots, ~400 on the busiest expert (4 tiles); K = 1024 (gate/up) and 2048 (down)
    check_layer(dev, 1024, 2048, 8, 2, qts, (512,), G.MATH_F32, seed=30, zipf=True)


def test_prefill_c3_shape_sampled(dev):
    # d 4096, f 14336, 8 experts, top-2, Q4_K, 512 Zipf-skewed tokens;
    # all 512 go through the GPU, 24 of them are checked against the oracle
    check_layer(dev, 4096, 14336, 8, 2, (G.Q4_K,) * 3, (512,), G.MATH_F32, seed=31, zipf=True, sample=24)


# Decode calls that compute their logits dispatch every expert that can be among a
# token's top k under a rigorous bound on the parallel logit, while the exact routing runs
# beside; the combine uses the exact ids and weights. Rows that tie exactly or within
# rounding force extra candidates; a router scaled so that most probabilities underflow
# makes every expert a candidate.
@pytest.mark.parametrize("gating", [G.GATING_LLAMA, G.GATING_MIXTRAL])
def test_speculative_candidates_cover_near_ties(dev, gating):
    def near_ties(R):
        R[2] = R[1]                                   # exact tie: lower id first
        R[4] = R[3] * np.float32(1 + 2 ** -20)        # within the parallel sum's error
        R[6] = R[5] + np.float32(1e-7)
        return R
    check_layer(dev, 4096, 512, 8, 2, (G.Q4_K,) * 3, (1, 2, 8, 33), G.MATH_PACKED, gating, seed=9,
                router_fn=near_ties)


def test_speculative_all_candidates_when_probabilities_underflow(dev):
    check_layer(dev, 256, 512, 8, 2, (G.Q4_K,) * 3, (1, 5, 16), G.MATH_PACKED, seed=10,
                router_fn=lambda R: R * np.float32(400.0))


def test_split_layout_matches_stacked(dev):
    check_layer(dev, 256, 512, 8, 2, (G.Q4_K,) * 3, (3,), G.MATH_PACKED, seed=4, split=True)


def test_fine_grained_c4_shape(dev):
    # d 2048, f 768, 128 experts, top-8, Q6_K gate/up, Q8_0 down,
    # 64 tokens, router logits uniform * 4 given directly
    check_layer(dev, 2048, 768, 128, 8, (G.Q6_K, G.Q6_K, G.Q8_0), (64,), G.MATH_PACKED, logits_scale=4.0, seed=5)


def test_reference_fixture_layer(dev):
    """The in-memory MoE GGUF of llama/mod.rs:1327-1401 (F32, d=32, ff=32, 4 experts)."""
    from tests.test_oracle_path import fixture_layer
    for math in (G.MATH_F32, G.MATH_PACKED):
        L = fixture_layer(1 if math == G.MATH_PACKED else 0)
        layer = G.MoeLayer(dev, 32, 32, 4, 2, L["router"], L["gate"], L["up"], L["down"], L["qtypes"], math=math)
        hs = np.random.default_rng(0).normal(0, 1, (12, 32)).astype(np.float32)
        out, ids, w = layer.feed_forward_batch(hs)
        wout, wids, ww = O.feed_forward_batch(L, hs)
        assert np.array_equal(ids, wids)
        assert np.allclose(out, wout, rtol=RTOL, atol=ATOL)
        # batched equals one token at a time (llama/mod.rs:1639-1688)
        for t in (0, 5, 11):
            o1 = layer.feed_forward_batch(hs[t:t + 1])[0]
            assert np.allclose(o1[0], out[t], rtol=1e-6, atol=1e-7)
        layer.release()


# ---------------- the L1 tier and error handling ----------------

def test_resident_layer_counts_a_hit_per_routed_expert():
    # ExpertCache::get on a resident expert is a hit (cache/mod.rs:18-137): one per
    # distinct expert a call routes to
    d, f, ne, k = 256, 512, 8, 2
    rng = np.random.default_rng(21)
    router, mats = make_layer(rng, d, f, ne, G.Q4_K, G.Q4_K)
    with G.Device(0, slab_bytes=64 << 20) as dev:
        layer = G.MoeLayer(dev, d, f, ne, k, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
        assert all(layer.is_resident(e) for e in range(ne))
        before = dev.slab_stats()
        _, ids, _ = layer.feed_forward_batch(rng.normal(0, 1, (3, d)).astype(np.float32))
        after = dev.slab_stats()
        assert after.hits - before.hits == len(np.unique(ids)) and after.misses == before.misses
        layer.release()


def test_small_slab_stages_experts_on_demand():
    d, f, ne, k = 256, 512, 8, 2
    rng = np.random.default_rng(12)
    router, mats = make_layer(rng, d, f, ne, G.Q4_K, G.Q4_K)
    per = sum(M.byte_size(G.Q4_K, f * d) for _ in range(3))
    # room for 4 experts: the most one call of n=2, top-2 can route to
    with G.Device(0, slab_bytes=4 * per + (1 << 16)) as small:
        layer = G.MoeLayer(small, d, f, ne, k, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
        resident = [layer.is_resident(e) for e in range(ne)]
        assert 0 < sum(resident) < ne
        L = oracle_layer(d, f, ne, k, router, mats, (G.Q4_K,) * 3, G.MATH_PACKED)
        for n in (1, 2, 1):
            hs = rng.normal(0, 1, (n, d)).astype(np.float32)
            out, ids, _ = layer.feed_forward_batch(hs)
            wout, wids, _ = O.feed_forward_batch(L, hs)
            assert np.array_equal(ids, wids) and np.allclose(out, wout, rtol=RTOL, atol=ATOL)
        st = small.slab_stats()
        assert st.misses > 0 and st.evictions > 0 and st.entries <= 4
        layer.evict(int(ids[0, 0]))
        assert not layer.is_resident(int(ids[0, 0]))
        layer.prefetch(int(ids[0, 0]))
        assert layer.is_resident(int(ids[0, 0]))
        with pytest.raises(G.CacheError):
            layer.forward_async(1, 1, 1)  # not every expert resident: refused before any launch


def test_small_slab_with_near_tie_candidates():
    # d = 4096 makes the logits' error bound wide enough that a near-tie expert is a
    # candidate of the speculative front end; with a slab of two experts it is not
    # resident, so a call that stages experts must run from its exact routing only
    d, f, ne, k = 4096, 512, 8, 2
    rng = np.random.default_rng(21)
    _, mats = make_layer(rng, d, f, ne, G.Q4_K, G.Q4_K)
    u = rng.normal(0, 1, d).astype(np.float32)
    u /= np.linalg.norm(u)
    r = rng.normal(0, 0.02, (ne, d)).astype(np.float32)
    r[0] = u                                                            # always first
    r[1] = 0.5 * u
    r[2] = r[1] + rng.normal(0, 1e-7, d).astype(np.float32)            # a near tie with expert 1
    router = np.ascontiguousarray(r.reshape(-1))
    per = sum(M.byte_size(G.Q4_K, f * d) for _ in range(3))
    with G.Device(0, slab_bytes=2 * per + (1 << 16)) as small:
        layer = G.MoeLayer(small, d, f, ne, k, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
        L = oracle_layer(d, f, ne, k, router, mats, (G.Q4_K,) * 3, G.MATH_PACKED)
        for step in range(6):
            hs = (rng.normal(0, 1, (1, d)) + 8 * u).astype(np.float32)
            say(f"near-tie small-slab step {step}")
            out, ids, _ = layer.feed_forward_batch(hs)
            wout, wids, _ = O.feed_forward_batch(L, hs)
            assert ids[0, 0] == 0 and ids[0, 1] in (1, 2)
            assert np.array_equal(ids, wids) and np.allclose(out, wout, rtol=RTOL, atol=ATOL)
        layer.release()


def test_bad_inputs_are_errors_not_crashes(dev):
    rng = np.random.default_rng(13)
    router, mats = make_layer(rng, 256, 512, 8, G.Q4_K, G.Q4_K)
    with pytest.raises(G.ConfigError):
        G.MoeLayer(dev, 256, 512, 8, 9, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
    with pytest.raises(G.ModelError):
        G.MoeLayer(dev, 256, 512, 8, 2, router, mats["gate"], mats["up"], mats["down"], (3, 3, 3))
    layer = G.MoeLayer(dev, 256, 512, 8, 2, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
    with pytest.raises(G.InferenceError):
        layer.feed_forward_batch(np.zeros((2, 100), np.float32))
    with pytest.raises(G.ModelError):
        dev.dequantize(G.Q4_K, np.zeros(100, np.uint8), 256)
    layer.release()
    with pytest.raises(G.InferenceError):
        layer.feed_forward_batch(np.zeros((1, 256), np.float32))
