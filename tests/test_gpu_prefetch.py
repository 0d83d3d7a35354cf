"""Predictor-driven prefetch into a slab too small for the layer (gmoe_prefetch_step):
predicted experts are queued for the context's staging thread and become resident, and
outputs are bit-identical to the same decode without prefetch (prefetch/mod.rs:1-10: a
guess can never change the answer; prefetch_engine_warms_experts_without_changing_logits,
llama/mod.rs:2116-2165). The step returns before the staging (PrefetchEngine::warm hands
its loads to a pool, prefetch/mod.rs:102-127): with the staging thread held, the predicted
experts stay queued, and a forward that routes to one takes it over and stages it itself.
Room for a prediction is made only by evicting experts the last two steps did not use."""
from __future__ import annotations

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd.predict import ExpertPredictor, PrefetchEngine
from tests.test_gpu_parity import bits, make_layer, say

pytestmark = pytest.mark.gpu

D, F, NE, K = 256, 512, 8, 2


def decode(prefetch: bool, steps: int = 60):
    rng = np.random.default_rng(0)
    router, mats = make_layer(rng, D, F, NE, G.Q4_K, G.Q4_K)
    expert_bytes = 3 * G.byte_size(G.Q4_K, D * F)
    dev = G.Device(0, slab_bytes=4 * (expert_bytes + 4096))  # four of the eight experts
    layer = G.MoeLayer(dev, D, F, NE, K, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
    eng = PrefetchEngine(dev, ExpertPredictor(NE), enabled=True, depth=K) if prefetch else None
    walk = np.random.default_rng(1)
    h = walk.normal(0, 1, D).astype(np.float32)
    outs, prev, last = [], [], []
    try:
        for step in range(steps):
            h = (0.9 * h + 0.45 * walk.normal(0, 1, D)).astype(np.float32)  # correlated steps
            out, ids, _ = layer.feed_forward_batch(h.reshape(1, D))
            outs.append((out.copy(), ids.copy()))
            if eng is not None:
                used = [int(x) for x in ids.reshape(-1)]
                last = eng.observe_step(layer, 0, prev, used, last)
                # the step returns with the predicted experts queued for the staging thread
                # (or already on their way); once it is idle they are resident
                for e in last:
                    assert layer.state(e) != G.moe.EXPERT_ABSENT, f"step {step}: predicted expert {e} dropped"
                dev.prefetch_wait()
                # room for a prediction is made only by evicting experts that neither this
                # step nor the one before used; when those and the predictions fill the
                # slab (four experts), a prediction that finds no room is dropped
                if len(set(used) | set(prev) | set(last)) <= 4:
                    for e in last:
                        assert layer.is_resident(e), f"step {step}: predicted expert {e} not staged"
                prev = used
        stats = eng.predictor_stats() if eng else None
        return outs, stats, (eng.launched, eng.skipped) if eng else None, dev.slab_stats()
    finally:
        layer.release()
        dev.close()


def test_prefetch_never_changes_outputs():
    base, _, _, s0 = decode(False)
    got, stats, (launched, skipped), s1 = decode(True)
    for i, ((o0, i0), (o1, i1)) in enumerate(zip(base, got)):
        assert np.array_equal(i0, i1) and np.array_equal(bits(o0), bits(o1)), f"step {i}"
    say(f"predictor precision {stats.precision():.2f} recall {stats.recall():.2f}, launched {launched}, "
        f"skipped {skipped}; forward misses {s0.misses} without, {s1.misses} with prefetch")
    # the predictor learns (llama/mod.rs:2158-2163: it must predict something) and every
    # in-layer prediction was either staged or already resident; whether prefetching
    # saves forward misses depends on the slab's size and the guesses' precision
    # (the last step's prediction is never scored)
    assert stats.correct > 0 and 0 < stats.correct + stats.wasted <= launched + skipped


def test_prefetch_step_refusals():
    dev = G.Device(0, slab_bytes=64 << 20)
    try:
        eng = PrefetchEngine(dev, ExpertPredictor(NE), enabled=True, depth=K)

        class Fake:
            id = 123
        with pytest.raises(G.InferenceError):
            eng.observe_step(Fake(), 0, [0], [1], [])
        assert PrefetchEngine(dev, ExpertPredictor(NE), enabled=False).observe_step(Fake(), 0, [0], [1], []) == []
    finally:
        dev.close()


def test_prefetch_step_returns_before_staging_and_a_forward_takes_the_queued_expert():
    from oracle import oracle as O
    from tests.test_gpu_parity import oracle_layer
    rng = np.random.default_rng(4)
    router, mats = make_layer(rng, D, F, NE, G.Q4_K, G.Q4_K)
    expert_bytes = 3 * G.byte_size(G.Q4_K, D * F)
    L = oracle_layer(D, F, NE, K, router, mats, (G.Q4_K,) * 3, G.MATH_PACKED)
    dev = G.Device(0, slab_bytes=4 * (expert_bytes + 4096))  # four of the eight experts
    layer = G.MoeLayer(dev, D, F, NE, K, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
    pred = ExpertPredictor(NE)
    eng = PrefetchEngine(dev, pred, enabled=True, depth=K)
    try:
        for trial, held in enumerate((True, False)):
            h = rng.normal(0, 1, (1, D)).astype(np.float32)
            _, want, _ = O.feed_forward_batch(L, h)  # the experts this token will route to
            a, b = (int(x) for x in want[0])
            for e in (a, b):
                layer.evict(e)
            # a learned transition x -> {a, b}: predict([x]) returns exactly a and b
            x = next(e for e in range(NE) if e not in (a, b))
            counts = np.zeros((NE, NE), np.uint32)
            counts[x, a], counts[x, b] = 5, 4
            pred.set_counts(counts)
            dev.prefetch_hold(held)
            got = eng.observe_step(layer, 0, [], [x], [])
            assert sorted(got) == sorted([a, b])
            if held:  # deterministically not staged yet when the step returns
                assert [layer.state(e) for e in (a, b)] == [G.moe.EXPERT_QUEUED] * 2
                assert not layer.is_resident(a) and not layer.is_resident(b)
            else:
                dev.prefetch_wait()
                assert layer.is_resident(a) and layer.is_resident(b)
            misses = dev.slab_stats().misses
            say(f"prefetch trial {trial} (held {held}): experts {a}, {b}")
            out, ids, _ = layer.feed_forward_batch(h)
            wout, wids, _ = O.feed_forward_batch(L, h)
            assert np.array_equal(ids, wids) and np.allclose(out, wout, rtol=1e-3, atol=1e-4)
            assert layer.is_resident(a) and layer.is_resident(b)
            # held: the forward took both off the queue and staged them (two misses); else hits
            assert dev.slab_stats().misses - misses == (2 if held else 0)
            dev.prefetch_hold(False)
            dev.prefetch_wait()
            assert all(layer.state(e) in (G.moe.EXPERT_ABSENT, G.moe.EXPERT_RESIDENT) for e in range(NE))
    finally:
        layer.release()
        dev.close()
