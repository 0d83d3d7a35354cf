"""A whole decode step on the GPU (gmoe_model_*, garuda_amd.DecodeModel) against the
oracle's restatement of logits_batch (oracle/model.py): a small packed model (C1's
shape class: d 256, GQA 8/2 of 32, 8 experts top-2 of 512) over three sequences, fed
their prompts one token per step and then decoding greedily. Logits within the layer
tolerance scaled to their size (the norms' sums and the dense products' K slices run in
another order than the reference's), next tokens equal wherever the top two logits are
apart by more than that. Refusals leave every sequence where it was."""
from __future__ import annotations

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd.attention import KvCache
from oracle.model import ModelOracle
from tests.test_gpu_parity import say
from tests.test_model_oracle import tiny_model

pytestmark = pytest.mark.gpu

D, NH, NKV, HD, F, NE, K, VOCAB, NL = 256, 8, 2, 32, 512, 8, 2, 512, 3


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=256 << 20)
    yield d
    d.close()


def gpu_model(dev, w, max_positions=64, max_seqs=4):
    layers, out, onorm, embd, (nh, nkv, hd) = w
    kv = KvCache(dev, len(layers), nh, nkv, hd, block_size=16, max_positions=max_positions, max_seqs=max_seqs)
    moe, dense = [], {n: [] for n in ("wq", "wk", "wv", "wo")}
    for L in layers:
        m = L["moe"]
        moe.append(G.MoeLayer(dev, m["d"], m["f"], m["ne"], m["k"], m["router"], m["gate"], m["up"], m["down"],
                              m["qtypes"]))
        for n in dense:
            qt, raw, r, c = L[n]
            dense[n].append(G.DenseWeight(dev, qt, r, c, raw))
    qt, raw, r, c = out
    head = G.DenseWeight(dev, qt, r, c, raw)
    model = G.DecodeModel(dev, kv, moe, dense["wq"], dense["wk"], dense["wv"], dense["wo"], head,
                          np.stack([L["attn_norm"] for L in layers]), np.stack([L["ffn_norm"] for L in layers]),
                          onorm, embd)
    return model, kv, moe, dense, head


def release(model, kv, moe, dense, head):
    model.close()
    for m in moe:
        m.release()
    for ws in dense.values():
        for x in ws:
            x.release()
    head.release()
    kv.close()


@pytest.fixture(scope="module")
def weights():
    return tiny_model(11, n_layers=NL, d=D, nh=NH, nkv=NKV, hd=HD, f=F, ne=NE, k=K, vocab=VOCAB)


def compare(got_next, got_logits, want_next, want_logits, what):
    scale = float(np.abs(want_logits).max())
    err = np.abs(got_logits - want_logits)
    assert np.allclose(got_logits, want_logits, rtol=1e-3, atol=1e-3 * scale), f"{what}: max err {err.max()}"
    for i, row in enumerate(want_logits):
        top = np.sort(row)[-2:]
        if top[1] - top[0] > 4e-3 * scale:
            assert got_next[i] == want_next[i], f"{what}: sequence {i} chose {got_next[i]}, not {want_next[i]}"


def test_decode_steps_match_the_reference_path(dev, weights):
    layers, out, onorm, embd, (nh, nkv, hd) = weights
    parts = gpu_model(dev, weights)
    model, kv = parts[0], parts[1]
    try:
        orc = ModelOracle(layers, out, onorm, embd, nh, nkv, hd, max_positions=64)
        seqs = [kv.open_seq() for _ in range(3)]
        rng = np.random.default_rng(3)
        prompt = rng.integers(0, VOCAB, (3, 6)).astype(np.uint32)
        toks = prompt[:, 0]
        for step in range(12):  # 6 prompt tokens, then greedy decoding
            say(f"model decode step {step}")
            gn, gl = model.decode_step(seqs, toks, want_logits=True)
            on, ol = orc.decode_step(seqs, toks)
            compare(gn, gl, on, ol, f"step {step}")
            toks = prompt[:, step + 1] if step + 1 < prompt.shape[1] else on
        for s in seqs:
            assert all(kv.seq_len(s, l) == 12 for l in range(NL))
        # a batch of one sequence, then the other two, continue the same caches
        gn, gl = model.decode_step([seqs[1]], toks[1:2], want_logits=True)
        on, ol = orc.decode_step([seqs[1]], toks[1:2])
        compare(gn, gl, on, ol, "single sequence")
    finally:
        release(*parts)


def test_refusals_leave_the_sequences_unchanged(dev, weights):
    parts = gpu_model(dev, weights, max_positions=3)
    model, kv, moe = parts[0], parts[1], parts[2]
    try:
        a, b = kv.open_seq(), kv.open_seq()
        model.decode_step([a, b], [1, 2])
        with pytest.raises(G.InvalidTokenError):
            model.decode_step([a, b], [1, VOCAB])
        with pytest.raises(G.InferenceError):
            model.decode_step([a, a], [1, 2])
        with pytest.raises(G.InferenceError):
            model.decode_step([a, 99], [1, 2])
        assert kv.seq_len(a, NL - 1) == 1 and kv.seq_len(b, NL - 1) == 1
        model.decode_step([a, b], [3, 4])
        model.decode_step([a], [5])
        with pytest.raises(G.CacheError):  # a's window of 3 positions is full
            model.decode_step([a, b], [6, 7])
        assert kv.seq_len(a, 0) == 3 and kv.seq_len(b, 0) == 2
        model.decode_step([b], [6])
        # an evicted expert: refused before any layer runs
        c = kv.open_seq()
        moe[1].evict(0)
        with pytest.raises(G.CacheError):
            model.decode_step([c], [1])
        assert kv.seq_len(c, 0) == 0
        moe[1].prefetch(0)
        model.decode_step([c], [1])
        assert kv.seq_len(c, NL - 1) == 1
    finally:
        release(*parts)
