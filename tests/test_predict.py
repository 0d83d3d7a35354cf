"""Expert predictor (garuda_amd/csrc/gmoe_predict.cpp through the C-ABI) against the
oracle's restatement (oracle/predict.py), and both against the reference's own tests
(garuda/src/predictor/mod.rs:140-205). Host code only."""
from __future__ import annotations

import numpy as np
import pytest

from garuda_amd.predict import ExpertPredictor, PredictStats
from oracle import predict as OP


@pytest.fixture(params=["library", "oracle"])
def make(request):
    return ExpertPredictor if request.param == "library" else OP.Predictor


def test_predicts_nothing_before_it_has_learned_anything(make):  # :140-145
    p = make(8)
    assert p.predict([0, 1], 2) == []
    assert p.predict([], 2) == []


def test_learns_a_repeated_transition(make):  # :147-157
    p = make(8)
    for _ in range(10):
        p.observe([0, 1], [3, 4])
    got = p.predict([0, 1], 2)
    assert len(got) == 2 and 3 in got and 4 in got


def test_prefers_the_more_frequent_successor(make):  # :159-168
    p = make(4)
    for _ in range(9):
        p.observe([0], [1])
    p.observe([0], [2])
    assert p.predict([0], 1) == [1]
    assert p.predict([0], 2) == [1, 2]


def test_ignores_out_of_range_expert_ids(make):  # :170-180
    p = make(4)
    p.observe([99], [1])
    p.observe([0], [99])
    assert p.predict([99], 2) == []
    assert p.predict([0], 2) == []


def test_saturating_counts_do_not_overflow():  # :182-191
    p = ExpertPredictor(2)
    c = np.zeros((2, 2), np.uint32)
    c[0, 0] = 2 ** 32 - 1
    p.set_counts(c)
    p.observe([0], [0])
    assert p.counts()[0, 0] == 2 ** 32 - 1
    assert p.predict([0], 1) == [0]
    o = OP.Predictor(2)
    o.counts[0][0] = OP.U32_MAX
    o.observe([0], [0])
    assert o.counts[0][0] == OP.U32_MAX and o.predict([0], 1) == [0]


def test_scoring_tracks_precision_and_recall():  # :193-204
    p = ExpertPredictor(8)
    p.score([1, 2], [2, 3])
    s = p.stats()
    assert (s.correct, s.wasted, s.missed) == (1, 1, 1)
    assert abs(s.precision() - 0.5) < 1e-9 and abs(s.recall() - 0.5) < 1e-9
    assert PredictStats(0, 0, 0).precision() == 0.0 and PredictStats(0, 0, 0).recall() == 0.0
    o = OP.Predictor(8)
    o.score([1, 2], [2, 3])
    assert (o.correct, o.wasted, o.missed) == (1, 1, 1)


@pytest.mark.parametrize("n,k", [(8, 2), (64, 6), (16, 16), (3, 5)])
def test_random_streams_match_the_oracle(n, k):
    rng = np.random.default_rng(n * 31 + k)
    lib, orc = ExpertPredictor(n), OP.Predictor(n)
    prev, last_l, last_o = [], [], []
    for step in range(400):
        # correlated steps: a random walk over expert ids, sometimes out of range or repeated
        base = int(rng.integers(0, n + 2))
        used = [int((base + int(rng.integers(0, 3))) % (n + 2)) for _ in range(int(rng.integers(1, k + 2)))]
        if last_l:
            lib.score(last_l, used)
            orc.score(last_o, used)
        if prev:
            lib.observe(prev, used)
            orc.observe(prev, used)
        last_l, last_o = lib.predict(used, k), orc.predict(used, k)
        assert last_l == last_o, f"step {step}"
        prev = used
    s = lib.stats()
    assert (s.correct, s.wasted, s.missed) == (orc.correct, orc.wasted, orc.missed)
    assert np.array_equal(lib.counts(), np.array(orc.counts, dtype=np.uint32))


def test_brute_force_ranking():
    # every ranking rule at once: ties broken to the lower id, zero scores dropped,
    # duplicates in `current` counted twice
    rng = np.random.default_rng(3)
    for _ in range(50):
        n = int(rng.integers(1, 7))
        c = rng.integers(0, 3, (n, n)).astype(np.uint32)
        p = ExpertPredictor(n)
        p.set_counts(c)
        cur = [int(x) for x in rng.integers(0, n + 1, int(rng.integers(0, 4)))]
        k = int(rng.integers(0, n + 2))
        score = {q: sum(int(c[x, q]) for x in cur if x < n) for q in range(n)}
        want = sorted([q for q in range(n) if score[q] > 0], key=lambda q: (-score[q], q))[:k] if cur and k else []
        assert p.predict(cur, k) == want
