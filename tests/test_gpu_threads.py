"""Concurrent callers on one context. InferenceBackend is Send + Sync (core/mod.rs:262) and
`hidden` can run beside decode (runtime/mod.rs:671-692), so the library serialises its
entry points per context and a call's results never depend on what another thread does
(the plugin contract's determinism, core/mod.rs:259-261): outputs are bit-identical to
the same calls made from one thread. With a slab too small for the layer, one thread's
forwards stage experts while another's prefetch steps queue and evict them; every
forward still routes and computes as the oracle does."""
from __future__ import annotations

import threading

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd.predict import ExpertPredictor, PrefetchEngine
from oracle import oracle as O
from tests.test_gpu_parity import bits, make_layer, oracle_layer, say

pytestmark = pytest.mark.gpu

D, F, NE, K = 256, 512, 8, 2


def run_threads(fns):
    errs = []

    def wrap(fn):
        try:
            fn()
        except BaseException as e:  # noqa: BLE001 - reported below
            errs.append(e)
    ts = [threading.Thread(target=wrap, args=(f,)) for f in fns]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=300)
        assert not t.is_alive(), "a thread did not finish"
    if errs:
        raise errs[0]


def test_two_threads_on_one_context_get_single_thread_results():
    rng = np.random.default_rng(30)
    router, mats = make_layer(rng, D, F, NE, G.Q4_K, G.Q4_K)
    dw = G.Q4_K, G.fill_gaussian(31, 512 * D, 0.0, 0.02)
    with G.Device(0, slab_bytes=256 << 20) as dev:
        layer = G.MoeLayer(dev, D, F, NE, K, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
        dense = G.DenseWeight(dev, G.Q4_K, 512, D, G.quantize(G.Q4_K, dw[1]))
        try:
            inputs = [rng.normal(0, 1, (n, D)).astype(np.float32) for n in (1, 8, 3, 1, 16, 2) * 4]
            want = [layer.feed_forward_batch(h) for h in inputs]
            want_dense = [dense.matmul_rows(h) for h in inputs]

            def worker(parity):
                for i in range(parity, len(inputs), 2):
                    out, ids, w = layer.feed_forward_batch(inputs[i])
                    assert np.array_equal(ids, want[i][1]) and np.array_equal(bits(w), bits(want[i][2]))
                    assert np.array_equal(bits(out), bits(want[i][0])), f"call {i}"
                    assert np.array_equal(bits(dense.matmul_rows(inputs[i])), bits(want_dense[i]))

            say("two threads, one resident layer and one dense weight")
            run_threads([lambda: worker(0), lambda: worker(1)])
        finally:
            dense.release()
            layer.release()


def test_forwards_beside_prefetch_steps_on_a_small_slab():
    rng = np.random.default_rng(32)
    router, mats = make_layer(rng, D, F, NE, G.Q4_K, G.Q4_K)
    L = oracle_layer(D, F, NE, K, router, mats, (G.Q4_K,) * 3, G.MATH_PACKED)
    expert_bytes = 3 * G.byte_size(G.Q4_K, D * F)
    with G.Device(0, slab_bytes=4 * (expert_bytes + 4096)) as dev:  # four of the eight experts
        layer = G.MoeLayer(dev, D, F, NE, K, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
        eng = PrefetchEngine(dev, ExpertPredictor(NE), enabled=True, depth=3)
        inputs = [rng.normal(0, 1, (1, D)).astype(np.float32) for _ in range(30)]
        wants = [O.feed_forward_batch(L, h) for h in inputs]
        try:
            def forwards():
                for h, (wout, wids, _) in zip(inputs, wants):
                    out, ids, _ = layer.feed_forward_batch(h)
                    assert np.array_equal(ids, wids) and np.allclose(out, wout, rtol=1e-3, atol=1e-4)

            def prefetches():
                r = np.random.default_rng(33)
                prev, last = [], []
                for _ in range(60):
                    used = [int(x) for x in r.choice(NE, K, replace=False)]
                    last = eng.observe_step(layer, 0, prev, used, last)
                    prev = used

            say("forwards beside prefetch steps")
            run_threads([forwards, prefetches])
            dev.prefetch_wait()
            assert dev.slab_stats().entries <= 4
        finally:
            layer.release()
