"""Pins the oracle's routing, softmax, synthetic-weight and feed-forward restatements.

Sources: simd/mod.rs:250-279 (softmax tests), router/mod.rs:121-217 (router
properties), weights/mod.rs:17-120 + models/l2_cache fixtures, llama/mod.rs:1258-2027
(the in-memory MoE GGUF fixture and its equivalence tests). Where the reference has
no known answer, an independent float64 computation or a brute-force sort fixes one.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---- softmax, simd/mod.rs:250-279 ----

def test_softmax_sums_to_one_and_survives_large_inputs():
    x = O.softmax([1000.0, 1000.5, 999.0])
    assert np.isfinite(x).all() and abs(x.sum() - 1.0) < 1e-5
    assert x[1] > x[0] > x[2]


def test_softmax_of_empty_and_fully_masked_is_not_nan():
    O.softmax(np.zeros(0, np.float32))
    m = O.softmax([-np.inf] * 3)
    assert np.isfinite(m).all() and abs(m.sum() - 1.0) < 1e-5


def test_a_nan_beside_a_finite_maximum_does_not_survive():
    x = O.softmax([1.0, np.nan, 2.0])
    assert np.isfinite(x).all() and abs(x.sum() - 1.0) < 1e-5


def test_softmax_matches_float64_reference():
    rng = np.random.default_rng(3)
    for _ in range(50):
        v = rng.normal(0, 3, 9).astype(np.float32)
        want = np.exp(v.astype(np.float64) - v.max())
        want /= want.sum()
        assert np.allclose(O.softmax(v), want, rtol=1e-6, atol=1e-7)


# ---- synthetic weights, weights/mod.rs:17-120 vs models/l2_cache fixtures ----

def test_synthesize_expert_reproduces_the_reference_l2_fixtures():
    fx = json.loads((GOLDEN / "l2_cache_experts.json").read_text())
    for eid, rec in fx.items():
        g, u, d = O.synthesize_expert(int(eid))
        raw = np.concatenate([g, u, d]).astype("<f4").tobytes()
        assert len(raw) == rec["bytes"]
        assert hashlib.sha256(raw).hexdigest() == rec["sha256"]
        assert g[:8].tolist() == rec["gate_head"]


# ---- gating ----

ROUTER_SEED = 0x6761_7275_6461_0006  # weights/mod.rs:48


def router_setup(d=128, ne=8):
    router = O.seeded(ROUTER_SEED, ne * d, O.lib().or_bound(d))
    h = np.sin(np.arange(d, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    return router, h


def route(kind, router, h, ne=8, k=2):
    logits = O.simd_matmul(router, ne, h.size, h, 1)
    return O.gate(kind, logits, k)


@pytest.mark.parametrize("kind", [1, 2, 3, 0])
def test_selects_top_k_distinct_experts_in_range(kind):  # router/mod.rs:132-145
    router, h = router_setup()
    ids, w = route(kind, router, h)
    assert len(set(ids.tolist())) == 2 and (ids < 8).all()


def test_mixtral_and_qwen_sum_to_one_deepseek_does_not_exceed_it():  # router/mod.rs:147-162
    router, h = router_setup()
    for kind in (1, 3, 0):
        _, w = route(kind, router, h)
        assert abs(w.sum() - 1.0) < 1e-5
    _, w = route(2, router, h)
    assert 0 < w.sum() <= 1 + 1e-5 and (w >= 0).all()


def test_ranking_is_descending_and_deterministic():  # router/mod.rs:164-172
    router, h = router_setup()
    a, wa = route(1, router, h)
    b, wb = route(1, router, h)
    assert (a == b).all() and (wa == wb).all()
    assert (np.diff(wa) <= 0).all()


def test_different_inputs_can_select_different_experts():  # router/mod.rs:174-193
    router, _ = router_setup()
    seen = set()
    for s in range(32):
        h = np.sin((s * 13 + np.arange(128)).astype(np.float32) * np.float32(0.21)).astype(np.float32)
        seen.update(route(1, router, h)[0].tolist())
    assert len(seen) > 1


def brute_llama_gate(scores, k):
    """llama/mod.rs:940-949 by brute force: stable sort of the softmax by value desc."""
    p = O.softmax(scores)
    order = sorted(range(len(p)), key=lambda i: -float(p[i]))  # Python's sort is stable
    top = order[:k]
    s = np.float32(-0.0)
    for i in top:
        s = np.float32(s + p[i])
    norm = np.float32(1.0) / s if s > 0 else np.float32(1.0) / np.float32(k)
    return np.array(top, np.uint32), np.array([np.float32(p[i] * norm) for i in top], np.float32)


def test_llama_gating_matches_brute_force_with_ties():
    rng = np.random.default_rng(11)
    for trial in range(300):
        ne = int(rng.choice([4, 8, 16, 128]))
        k = int(rng.integers(1, min(ne, 8) + 1))
        v = rng.normal(0, 2, ne).astype(np.float32)
        if trial % 3 == 0:  # exact ties decide by lower id
            v[rng.integers(0, ne, ne // 2)] = v[0]
        ids, w = O.gate(0, v, k)
        bi, bw = brute_llama_gate(v, k)
        assert (ids == bi).all()
        assert np.array_equal(w.view(np.uint32), bw.view(np.uint32))


def test_router_mixtral_tie_breaks_on_lower_id():
    ids, w = O.gate(1, np.array([0.5, 1.0, 1.0, 0.2], np.float32), 2)
    assert ids.tolist() == [1, 2] and np.allclose(w, [0.5, 0.5])


def softmax64(v):
    v = np.asarray(v, np.float64)
    e = np.exp(v - v.max())
    return e / e.sum()


def test_deepseek_weights_are_the_full_softmax_without_renormalisation():
    """router/mod.rs:74-76, :99-101: DeepSeek softmaxes over every expert, keeps the top
    k by probability (partial_cmp descending, ties to the lower id, :83-88) and leaves
    the kept probabilities as they are. Pinned three ways: each weight is the full
    softmax's entry bit for bit, within float32 rounding of a float64 softmax, and the
    weights fall short of 1 by the probability left out."""
    rng = np.random.default_rng(17)
    for trial in range(400):
        ne = int(rng.choice([4, 8, 16, 64, 128]))
        k = int(rng.integers(1, min(ne, 8) + 1))
        v = rng.normal(0, 1.5, ne).astype(np.float32)
        if trial % 4 == 0:
            v[rng.integers(0, ne, ne // 3)] = v[1]  # exact ties go to the lower id
        ids, w = O.gate(2, v, k)
        p = O.softmax(v)
        order = sorted(range(ne), key=lambda i: (-float(p[i]), i))
        assert ids.tolist() == order[:k]
        assert np.array_equal(w.view(np.uint32), p[ids].view(np.uint32))
        p64 = softmax64(v)[ids]
        assert (np.abs(w.astype(np.float64) - p64) <= 1e-7 + 1e-6 * p64).all()
        left = float(np.sort(p)[::-1][k]) if k < ne else 0.0
        s = float(np.float32(sum(np.float32(x) for x in w)))
        if left > 1e-6:
            assert s <= 1.0 - left / 2, (trial, s, left)
        else:
            assert s <= 1.0 + 1e-6


def test_deepseek_closed_form_and_qwen_is_its_renormalisation():
    """Logits (2, 1, 0, -1), k = 2: the weights are e^2/Z and e^1/Z with Z = e^2 + e + 1 +
    1/e (0.6439, 0.2369); QwenMoe keeps the same experts and divides by their sum
    (router/mod.rs:102-115)."""
    v = np.array([2.0, 1.0, 0.0, -1.0], np.float32)
    ids, w = O.gate(2, v, 2)
    z = np.exp(2.0) + np.exp(1.0) + 1.0 + np.exp(-1.0)
    assert ids.tolist() == [0, 1]
    assert np.allclose(w, [np.exp(2.0) / z, np.exp(1.0) / z], rtol=1e-6, atol=0)
    assert 0.88 < float(w.sum()) < 0.881
    rng = np.random.default_rng(23)
    for _ in range(200):
        ne = int(rng.choice([8, 16, 128]))
        k = int(rng.integers(1, min(ne, 8) + 1))
        v = rng.normal(0, 2, ne).astype(np.float32)
        ids_d, w_d = O.gate(2, v, k)
        ids_q, w_q = O.gate(3, v, k)
        assert (ids_d == ids_q).all()
        s = np.float32(-0.0)
        for x in w_d:
            s = np.float32(s + x)
        assert np.array_equal(w_q.view(np.uint32), (w_d / s).astype(np.float32).view(np.uint32))


# ---- the feed-forward layer on the reference's in-memory MoE fixture ----

def gen(seed, n):
    """llama/mod.rs:1290-1299 (usize arithmetic, wrapping)."""
    i = np.arange(n, dtype=np.uint64)
    h = (np.uint64(seed) * np.uint64(2_654_435_761) + i * np.uint64(40_503))
    return ((h % np.uint64(2000)).astype(np.float32) / np.float32(2000.0) - np.float32(0.5)).astype(np.float32)


def fixture_layer(packed=0):
    """Layer 0's FFN of build_gguf (llama/mod.rs:1327-1401): d=32, ff=32, 4 experts,
    top-2, F32. Seeds follow the builder's counter: token_embd 1, output_norm 2,
    output 3, then per layer 7 tensors (attn_norm..ffn_gate_inp = 4..10) and the
    three stacked expert tensors 11, 12, 13."""
    d, ff, ne = 32, 32, 4
    router = gen(10, d * ne)
    gate = gen(11, ne * ff * d)
    up = gen(12, ne * ff * d)
    down = gen(13, ne * d * ff)
    as_u8 = lambda a: a.astype("<f4").view(np.uint8)
    return dict(d=d, f=ff, ne=ne, k=2, gating=0, combine=0, packed=packed, router=router,
                qtypes=(O.F32, O.F32, O.F32), gate=as_u8(gate), up=as_u8(up), down=as_u8(down))


def f64_ffn(layer, hs, w_gate, w_up, w_down):
    """Independent float64 restatement of one MoE FFN with the oracle's routing."""
    d, f, ne, k = layer["d"], layer["f"], layer["ne"], layer["k"]
    out = np.zeros((hs.shape[0], d))
    for t in range(hs.shape[0]):
        logits = O.simd_matmul(layer["router"], ne, d, hs[t], 1)
        ids, w = O.gate(layer["gating"], logits, k)
        for e, wt in sorted(zip(ids.tolist(), w.tolist())):
            x = hs[t].astype(np.float64)
            g = w_gate[e] @ x
            u = w_up[e] @ x
            h = g / (1 + np.exp(-g)) * u
            out[t] += wt * (w_down[e] @ h)
    return out


def test_fixture_ffn_matches_float64_restatement():
    L = fixture_layer()
    rng = np.random.default_rng(0)
    hs = rng.normal(0, 1, (6, 32)).astype(np.float32)
    out, ids, w = O.feed_forward_batch(L, hs)
    deq = lambda a, rows, cols: a.view("<f4").astype(np.float64).reshape(4, rows, cols)
    want = f64_ffn(L, hs, deq(L["gate"], 32, 32), deq(L["up"], 32, 32), deq(L["down"], 32, 32))
    assert np.allclose(out, want, rtol=1e-5, atol=1e-6)


def test_batched_layer_matches_each_token_alone():
    """llama/mod.rs:1639-1688 at the layer: one call over n tokens equals n calls."""
    L = fixture_layer()
    hs = np.random.default_rng(1).normal(0, 1, (7, 32)).astype(np.float32)
    out, ids, w = O.feed_forward_batch(L, hs)
    for t in range(7):
        o1, i1, w1 = O.feed_forward_batch(L, hs[t:t + 1])
        assert np.array_equal(o1[0].view(np.uint32), out[t].view(np.uint32))
        assert (i1[0] == ids[t]).all()


def test_packed_path_is_f32_path_for_f32_weights():
    """llama/mod.rs:1964-2010: F32 has no int8 kernel, so mmap and f32 agree."""
    hs = np.random.default_rng(2).normal(0, 1, (3, 32)).astype(np.float32)
    a = O.feed_forward_batch(fixture_layer(0), hs)[0]
    b = O.feed_forward_batch(fixture_layer(1), hs)[0]
    assert np.abs(a - b).max() < 1e-3


def test_rank_order_combine_differs_only_in_add_order():
    L = fixture_layer()
    L2 = dict(L, combine=1)
    hs = np.random.default_rng(3).normal(0, 1, (5, 32)).astype(np.float32)
    a = O.feed_forward_batch(L, hs)[0]
    b = O.feed_forward_batch(L2, hs)[0]
    assert np.allclose(a, b, rtol=1e-6, atol=1e-6)


def test_q4k_packed_layer_tracks_full_layer_within_int8_error():
    """The packed path differs from the f32 one only by int8 activations (~1% here)."""
    from garuda_amd import moe as M
    d, f, ne = 256, 512, 8
    rng = np.random.default_rng(4)
    router = rng.normal(0, 0.02, ne * d).astype(np.float32)
    mats = {n: M.quantize(O.Q4_K, rng.normal(0, 0.02, ne * r * c).astype(np.float32))
            for n, r, c in (("gate", f, d), ("up", f, d), ("down", d, f))}
    L = dict(d=d, f=f, ne=ne, k=2, router=router, qtypes=(O.Q4_K,) * 3, **mats)
    hs = rng.normal(0, 1, (4, d)).astype(np.float32)
    a, ia, _ = O.feed_forward_batch(dict(L, packed=1), hs)
    b, ib, _ = O.feed_forward_batch(dict(L, packed=0), hs)
    assert (ia == ib).all()
    rel = np.linalg.norm(a - b) / np.linalg.norm(b)
    assert 1e-5 < rel < 0.05


# ---- gating on non-finite logits ----
# simd::softmax falls back to uniform when the maximum or the sum is not finite
# (simd/mod.rs:132-158), which fixes llama, DeepSeek and Qwen gating on NaN and +-inf:
# uniform probabilities, ranked by id. Mixtral ranks the raw logits with partial_cmp,
# which is no order once a value is NaN (router/mod.rs:83-88: Rust's sort_by then gives
# an unspecified order or panics): this build ranks a NaN after every number, NaNs among
# themselves by id (parity unpinned: nothing in the reference fixes that case).

def _brute_router_topk(scores, k):
    s = np.asarray(scores, np.float32)
    order = sorted(range(s.size), key=lambda i: (bool(np.isnan(s[i])), 0.0 if np.isnan(s[i]) else -float(s[i]), i))
    return order[:k]


def test_softmax_gatings_are_uniform_on_nan_or_infinity():
    for bad in (np.nan, np.inf):
        scores = np.array([0.3, bad, -1.0, 2.0, 0.5], np.float32)
        for kind in (0, 2, 3):  # llama, DeepSeek, Qwen
            ids, w = O.gate(kind, scores, 2)
            assert ids.tolist() == [0, 1], (kind, bad)  # equal probabilities: lower ids first
            want = {0: 0.5, 2: 0.2, 3: 0.5}[kind]  # llama/Qwen renormalise, DeepSeek keeps 1/ne
            assert np.allclose(w, want), (kind, bad, w)
    # -inf beside finite values is an ordinary masked logit: exp(-inf) = 0
    ids, w = O.gate(0, np.array([0.3, -np.inf, 2.0], np.float32), 2)
    assert ids.tolist() == [2, 0] and w[1] > 0


def test_mixtral_ranks_nan_after_every_number():
    ids, w = O.gate(1, np.array([1.0, np.nan, 2.0], np.float32), 2)
    assert ids.tolist() == [2, 0]
    assert np.allclose(w, np.exp([0.0, -1.0]) / np.exp([0.0, -1.0]).sum())
    # +-inf are numbers: +inf first, -inf after every finite value but before NaN
    ids, w = O.gate(1, np.array([np.nan, -np.inf, 0.5, np.inf], np.float32), 3)
    assert ids.tolist() == [3, 2, 1]
    assert np.allclose(w, 1.0 / 3)  # softmax over [inf, 0.5, -inf]: the maximum is not finite
    # fewer than k numbers: the NaNs follow by id, and the kept NaN makes softmax uniform
    ids, w = O.gate(1, np.array([np.nan, 3.0, np.nan, np.nan], np.float32), 3)
    assert ids.tolist() == [1, 0, 2] and np.allclose(w, 1.0 / 3)
    rng = np.random.default_rng(8)
    for _ in range(300):
        ne = int(rng.integers(2, 40))
        s = rng.normal(0, 2, ne).astype(np.float32)
        s[rng.random(ne) < 0.3] = np.nan
        s[rng.random(ne) < 0.1] = np.inf
        s[rng.random(ne) < 0.1] = -np.inf
        s[rng.random(ne) < 0.2] = s[0]  # ties
        k = int(rng.integers(1, ne + 1))
        ids, _ = O.gate(1, s, k)
        assert ids.tolist() == _brute_router_topk(s, k)
