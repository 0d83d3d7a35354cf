"""The attention oracle (oracle/attention.py) pinned by the reference's rope tests
(garuda/src/simd/mod.rs:282-299) and by closed forms. Host only."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as OA


def test_rope_is_norm_preserving():  # simd/mod.rs:282-289
    v = np.array([0.3, -1.2, 0.7, 2.0], np.float32)
    r = OA.rope(v, 5, 10_000.0)
    assert abs(np.linalg.norm(v) - np.linalg.norm(r)) < 1e-5


def test_rope_at_position_zero_is_identity():  # simd/mod.rs:291-299
    v = np.array([0.3, -1.2, 0.7, 2.0], np.float32)
    assert np.allclose(OA.rope(v, 0, 10_000.0), v, atol=1e-6)


@pytest.mark.parametrize("hd,pos", [(4, 3), (64, 100), (128, 2047)])
def test_rope_of_unit_pairs_is_cos_sin_of_the_angle(hd, pos):
    v = np.zeros(hd, np.float32)
    v[0::2] = 1.0
    r = OA.rope(v, pos, 10_000.0)
    i = np.arange(hd // 2)
    ang = pos * (1.0 / 10_000.0 ** (2.0 * i / hd))
    assert np.allclose(r[0::2], np.cos(ang), atol=2e-4) and np.allclose(r[1::2], np.sin(ang), atol=2e-4)


def test_one_position_returns_its_value():
    o = OA.KvOracle(1, 4, 2, 8)
    rng = np.random.default_rng(0)
    q, k, v = rng.normal(size=32), rng.normal(size=16), rng.normal(size=16)
    out = o.attend_one(0, 0, q, k, v)
    group = 2
    for h in range(4):
        assert np.allclose(out[h * 8:(h + 1) * 8], v[(h // group) * 8:(h // group + 1) * 8].astype(np.float32))


def test_equal_scores_average_the_values():
    o = OA.KvOracle(1, 2, 1, 4)
    rng = np.random.default_rng(1)
    vals = []
    for _ in range(5):
        v = rng.normal(size=4).astype(np.float32)
        vals.append(v)
        out = o.attend_one(0, 0, np.zeros(8), np.zeros(4), v)  # q = 0: every score is 0
    assert np.allclose(out[:4], np.mean(vals, axis=0)) and np.allclose(out[4:], np.mean(vals, axis=0))


def test_brute_force_gqa_and_window():
    rng = np.random.default_rng(2)
    nh, nkv, hd, win = 6, 2, 8, 5
    o = OA.KvOracle(2, nh, nkv, hd, sliding_window=win)
    K, V = [], []
    for pos in range(12):
        q, k, v = rng.normal(size=nh * hd), rng.normal(size=nkv * hd), rng.normal(size=nkv * hd)
        out = o.attend_one(1, 3, q, k, v)
        qr = np.concatenate([OA.rope(q[h * hd:(h + 1) * hd], pos, 1e4) for h in range(nh)])
        K.append(np.concatenate([OA.rope(k[h * hd:(h + 1) * hd], pos, 1e4) for h in range(nkv)]))
        V.append(v.astype(np.float32))
        start = max(0, pos + 1 - win)
        for h in range(nh):
            kh = h // (nh // nkv)
            s = [float(np.dot(qr[h * hd:(h + 1) * hd], K[j][kh * hd:(kh + 1) * hd])) / np.sqrt(hd)
                 for j in range(start, pos + 1)]
            p = np.exp(np.array(s) - max(s))
            p /= p.sum()
            want = sum(p[j - start] * V[j][kh * hd:(kh + 1) * hd] for j in range(start, pos + 1))
            assert np.allclose(out[h * hd:(h + 1) * hd], want, atol=1e-5)
    assert o.seq_len(3, 1) == 12 and o.seq_len(3, 0) == 0


def test_context_window_is_enforced():
    o = OA.KvOracle(1, 1, 1, 4, max_positions=2)
    for _ in range(2):
        o.attend_one(0, 0, np.ones(4), np.ones(4), np.ones(4))
    with pytest.raises(ValueError):
        o.attend_one(0, 0, np.ones(4), np.ones(4), np.ones(4))


def nan_inf_case(bad):
    """Inputs whose scores hit the reference softmax's fallback: with bad = "nan" the key at
    position 2 of kv head 0 carries a NaN (every later score of that head is NaN); with
    bad = "inf" the key at position 0 is (1e30, 0, 0, 0) and the query at position 1 is
    rotated back onto it, so its f32 score 1e60 / 2 overflows to +inf. Heads of 4 values
    (2 query heads, 1 kv head) or 8 (4 query heads, 2 kv heads). Returns the steps as
    (q, k, v) triples."""
    rng = np.random.default_rng(3)
    steps = []
    if bad == "nan":
        nh, nkv, hd = 4, 2, 8
        for pos in range(6):
            q, k, v = rng.normal(size=nh * hd), rng.normal(size=nkv * hd), rng.normal(size=nkv * hd)
            if pos == 2:
                k[0] = np.nan
            steps.append((q, k, v))
        return (nh, nkv, hd), steps
    nh, nkv, hd = 2, 1, 4
    k0 = np.array([1e30, 0, 0, 0])
    q1 = np.array([np.cos(-1.0) * 1e30, np.sin(-1.0) * 1e30, 0, 0])  # rope at position 1 turns it by +1 rad
    steps.append((rng.normal(size=nh * hd), k0, rng.normal(size=nkv * hd)))
    steps.append((np.concatenate([q1, q1]), rng.normal(size=nkv * hd), rng.normal(size=nkv * hd)))
    return (nh, nkv, hd), steps


def test_a_nan_or_infinite_score_gives_uniform_weights():
    """simd::softmax (simd/mod.rs:132-158): a NaN score poisons the sum and +inf makes the
    maximum non-finite; both fall back to uniform weights, so the context is the mean of
    the span's values. Only the kv head whose key carries the bad value is affected."""
    for bad in ("nan", "inf"):
        (nh, nkv, hd), steps = nan_inf_case(bad)
        o = OA.KvOracle(1, nh, nkv, hd)
        vals = []
        for pos, (q, k, v) in enumerate(steps):
            vals.append(v.astype(np.float32))
            out = o.attend_one(0, 0, q, k, v)
            if (bad == "nan" and pos >= 2) or (bad == "inf" and pos == 1):
                mean0 = np.mean([x[:hd] for x in vals], axis=0)
                for h in range(nh // nkv):  # the query heads of kv head 0
                    assert np.allclose(out[h * hd:(h + 1) * hd], mean0, atol=1e-6), (bad, pos, h)
                assert np.isfinite(out).all()
        if bad == "inf":  # without the fallback position 0 would take all the weight
            assert not np.allclose(out[:hd], vals[0][:hd], atol=1e-3)

