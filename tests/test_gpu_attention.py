"""Decode attention over the paged KV cache (gmoe_kv_*, gmoe_attention*) against the
oracle's attend_one / KVCacheState restatement (oracle/attention.py), within the layer
tolerance (rtol 1e-3, atol 1e-4): single sequences across page and chunk boundaries,
continuous batches of sequences at different lengths, prompts prefilled in one call,
sliding windows, the C5 head shape, refusals, page reuse, and the async form."""
from __future__ import annotations

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd.attention import KvCache
from oracle.attention import KvOracle
from tests.test_gpu_dense import _hip
from tests.test_gpu_parity import ATOL, RTOL, bits, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=64 << 20)
    yield d
    d.close()


def check(got, want, what):
    err = np.abs(got - want)
    assert np.allclose(got, want, rtol=RTOL, atol=ATOL), f"{what}: max err {err.max()}"


def test_one_sequence_across_pages_and_chunks(dev):
    nh, nkv, hd = 8, 2, 64
    rng = np.random.default_rng(0)
    with KvCache(dev, 2, nh, nkv, hd, block_size=16, max_positions=600, max_seqs=2) as kv:
        o = KvOracle(2, nh, nkv, hd, max_positions=600)
        s = kv.open_seq()
        for step in range(530):  # crosses 16-position pages and 256-position chunks
            q, k, v = rng.normal(size=(1, nh * hd)), rng.normal(size=(1, nkv * hd)), rng.normal(size=(1, nkv * hd))
            got = kv.attention(1, [s], q, k, v)
            want = o.attention(1, [s], q, k, v)
            if step % 37 == 0 or step in (255, 256, 257, 511, 512, 529):
                say(f"one sequence, step {step}")
                check(got, want, f"step {step}")
        assert kv.seq_len(s, 1) == 530 and kv.seq_len(s, 0) == 0


def test_continuous_batch_prefill_and_window(dev):
    nh, nkv, hd = 8, 8, 32
    rng = np.random.default_rng(1)
    with KvCache(dev, 1, nh, nkv, hd, block_size=8, max_positions=400, sliding_window=100, max_seqs=4) as kv:
        o = KvOracle(1, nh, nkv, hd, max_positions=400, sliding_window=100)
        seqs = [kv.open_seq() for _ in range(3)]
        # prompts of different lengths, each prefilled in one call (entries in order)
        for s, plen in zip(seqs, (5, 130, 17)):
            ids = [s] * plen
            q, k, v = (rng.normal(size=(plen, w)) for w in (nh * hd, nkv * hd, nkv * hd))
            check(kv.attention(0, ids, q, k, v), o.attention(0, ids, q, k, v), f"prefill seq {s}")
        # decode steps over all three at once, then with one sequence twice per call
        for step in range(60):
            ids = seqs if step % 3 else seqs + [seqs[1]]
            n = len(ids)
            q, k, v = (rng.normal(size=(n, w)) for w in (nh * hd, nkv * hd, nkv * hd))
            check(kv.attention(0, ids, q, k, v), o.attention(0, ids, q, k, v), f"decode step {step}")
        for s in seqs:
            assert kv.seq_len(s) == o.seq_len(s)


@pytest.mark.parametrize("nh,nkv,hd", [(32, 2, 256), (16, 2, 96), (8, 1, 128)])
def test_wide_heads_and_groups(dev, nh, nkv, hd):
    # heads wider than 128 (the wide-head kernel), widths not a multiple of 16, and
    # groups whose (head, column) items exceed one pass of the workgroup
    rng = np.random.default_rng(hd)
    with KvCache(dev, 1, nh, nkv, hd, block_size=16, max_positions=300, max_seqs=2) as kv:
        o = KvOracle(1, nh, nkv, hd, max_positions=300)
        seqs = [kv.open_seq() for _ in range(2)]
        ids = [seqs[0]] * 150 + [seqs[1]] * 70  # prompts across chunks, one call
        q, k, v = (rng.normal(size=(len(ids), w)) for w in (nh * hd, nkv * hd, nkv * hd))
        say(f"wide heads nh={nh} nkv={nkv} hd={hd}: prefill")
        check(kv.attention(0, ids, q, k, v), o.attention(0, ids, q, k, v), "prefill")
        for step in range(3):
            q, k, v = (rng.normal(size=(2, w)) for w in (nh * hd, nkv * hd, nkv * hd))
            check(kv.attention(0, seqs, q, k, v), o.attention(0, seqs, q, k, v), f"decode {step}")


def test_c5_head_shape(dev):
    # 32 query heads on 8 kv heads of 128, eight sequences
    nh, nkv, hd = 32, 8, 128
    rng = np.random.default_rng(2)
    with KvCache(dev, 1, nh, nkv, hd, block_size=16, max_positions=2048, max_seqs=8) as kv:
        o = KvOracle(1, nh, nkv, hd, max_positions=2048)
        seqs = [kv.open_seq() for _ in range(8)]
        ids = [s for s in seqs for _ in range(40)]  # 40-token prompts, one call
        q, k, v = (rng.normal(size=(len(ids), w)) for w in (nh * hd, nkv * hd, nkv * hd))
        check(kv.attention(0, ids, q, k, v), o.attention(0, ids, q, k, v), "c5 prefill")
        for step in range(3):
            q, k, v = (rng.normal(size=(8, w)) for w in (nh * hd, nkv * hd, nkv * hd))
            check(kv.attention(0, seqs, q, k, v), o.attention(0, seqs, q, k, v), f"c5 decode {step}")


def test_refusals_and_page_reuse(dev):
    nh, nkv, hd = 4, 2, 16
    rng = np.random.default_rng(3)
    with KvCache(dev, 1, nh, nkv, hd, block_size=4, max_positions=10, max_seqs=2, max_pages=4) as kv:
        a = kv.open_seq()
        b = kv.open_seq()
        with pytest.raises(G.CacheError):
            kv.open_seq()  # both sequence slots taken
        mk = lambda n: (rng.normal(size=(n, nh * hd)), rng.normal(size=(n, nkv * hd)), rng.normal(size=(n, nkv * hd)))
        kv.attention(0, [a] * 10, *mk(10))  # 3 pages
        with pytest.raises(G.CacheError):
            kv.attention(0, [a], *mk(1))  # context window of 10 exhausted
        with pytest.raises(G.CacheError):
            kv.attention(0, [b] * 5, *mk(5))  # needs 2 pages, 1 free: refused, nothing changes
        assert kv.seq_len(b) == 0
        with pytest.raises(G.InferenceError):
            kv.attention(0, [7], *mk(1))
        kv.close_seq(a)  # its pages return to the pool
        o = KvOracle(1, nh, nkv, hd, max_positions=10)
        q, k, v = mk(8)
        check(kv.attention(0, [b] * 8, q, k, v), o.attention(0, [b] * 8, q, k, v), "reused pages")


def test_async_matches_sync(dev):
    import ctypes as C
    hip = _hip()
    nh, nkv, hd, n = 8, 2, 64, 4
    rng = np.random.default_rng(4)
    qs, ks, vs = [rng.normal(size=(n, w)).astype(np.float32) for w in (nh * hd, nkv * hd, nkv * hd)]
    with KvCache(dev, 1, nh, nkv, hd) as A, KvCache(dev, 1, nh, nkv, hd) as B:
        sa = [A.open_seq() for _ in range(n)]
        sb = [B.open_seq() for _ in range(n)]
        want = A.attention(0, sa, qs, ks, vs)
        bufs = [C.c_void_p() for _ in range(4)]
        for b, a in zip(bufs, (qs, ks, vs, want)):
            assert hip.hipMalloc(C.byref(b), a.nbytes) == 0
        st = C.c_void_p()
        assert hip.hipStreamCreate(C.byref(st)) == 0
        try:
            for b, a in zip(bufs[:3], (qs, ks, vs)):
                assert hip.hipMemcpy(b, a.ctypes.data, a.nbytes, 1) == 0
            B.attention_async(0, sb, bufs[0].value, bufs[1].value, bufs[2].value, bufs[3].value, st.value)
            assert hip.hipStreamSynchronize(st) == 0
            got = np.empty_like(want)
            assert hip.hipMemcpy(got.ctypes.data, bufs[3], got.nbytes, 2) == 0
            assert np.array_equal(bits(got), bits(want))
        finally:
            hip.hipStreamDestroy(st)
            for b in bufs:
                hip.hipFree(b)


@pytest.mark.parametrize("bad", ["nan", "inf"])
def test_nan_or_infinite_score_gives_uniform_weights(dev, bad):
    # simd::softmax falls back to uniform weights on a NaN or +inf score (simd/mod.rs:132-158)
    from tests.test_attention_oracle import nan_inf_case
    (nh, nkv, hd), steps = nan_inf_case(bad)
    with KvCache(dev, 1, nh, nkv, hd, block_size=4, max_positions=64, max_seqs=1) as kv:
        o = KvOracle(1, nh, nkv, hd, max_positions=64)
        s = kv.open_seq()
        for pos, (q, k, v) in enumerate(steps):
            say(f"{bad} score, position {pos}")
            got = kv.attention(0, [s], q[None], k[None], v[None])
            want = o.attention(0, [s], q[None], k[None], v[None])
            assert np.isfinite(got).all()
            check(got, want, f"{bad} position {pos}")
