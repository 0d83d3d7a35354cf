"""Pins of the decode-step oracle (oracle/model.py) on the CPU: the reference's own tests
for the pieces it adds (greedy sampling, runtime/mod.rs:1112-1120; rmsnorm of an empty
row, simd/mod.rs:301-304), closed forms, and properties the reference asserts of
logits_batch (a batch of sequences computes what each would alone)."""
from __future__ import annotations

import numpy as np
import pytest

from garuda_amd import moe as M
from oracle import oracle as O
from oracle.model import ModelOracle, greedy, norm, rmsnorm


def test_greedy_takes_the_argmax():
    # runtime/mod.rs:1112-1120
    assert greedy(np.array([0.1, 5.0, -2.0, 4.9], dtype=np.float32)) == 1


def test_greedy_ties_nan_and_infinities():
    assert greedy(np.array([1.0, 3.0, 3.0, 2.0], dtype=np.float32)) == 1  # the first of equal maxima
    assert greedy(np.array([np.nan, 1.0, np.nan], dtype=np.float32)) == 1  # NaN never wins
    assert greedy(np.array([-np.inf, -np.inf], dtype=np.float32)) == 0  # nothing beats the -inf start
    assert greedy(np.array([np.nan, np.nan], dtype=np.float32)) == 0
    assert greedy(np.array([-np.inf, -1e30, np.inf], dtype=np.float32)) == 2


def test_rmsnorm_closed_forms():
    # simd/mod.rs:301-304: an empty row is left alone
    assert rmsnorm(np.zeros(0, dtype=np.float32), 1e-5).size == 0
    # [3, 4]: mean of squares 12.5
    got = rmsnorm(np.array([3.0, 4.0], dtype=np.float32), 0.0)
    want = np.array([3.0, 4.0]) / np.sqrt(12.5)
    assert np.allclose(got, want, rtol=1e-6)
    # a constant row c: c / sqrt(c^2 + eps)
    c, eps = np.float32(0.25), 1e-5
    got = rmsnorm(np.full(64, c, dtype=np.float32), eps)
    assert np.allclose(got, c / np.sqrt(c * c + eps), rtol=1e-6)
    # zeros stay zeros with eps > 0; the weight multiplies afterwards
    assert not rmsnorm(np.zeros(8, dtype=np.float32), 1e-5).any()
    w = np.arange(1, 5, dtype=np.float32)
    assert np.array_equal(norm(np.array([3.0, 4.0, 3.0, 4.0], dtype=np.float32), w, 0.0),
                          (rmsnorm(np.array([3.0, 4.0, 3.0, 4.0], dtype=np.float32), 0.0) * w).astype(np.float32))


def test_rmsnorm_sums_in_order():
    # the f32 sum of squares runs left to right: a large square first swallows the small ones
    x = np.array([4096.0] + [1.0] * 16, dtype=np.float32)
    seq = np.float32(0.0)
    for v in x:
        seq = np.float32(seq + np.float32(v * v))
    mean = np.float32(seq / np.float32(x.size))
    assert np.array_equal(rmsnorm(x, 0.0), (x * np.float32(1.0 / np.sqrt(mean))).astype(np.float32))


def tiny_model(seed, n_layers=2, d=256, nh=8, nkv=2, hd=32, f=256, ne=4, k=2, vocab=64):
    """Weights of a small packed model (Q4_K everywhere, Q6_K head) for the oracle."""
    rng = np.random.default_rng(seed)

    def q(qt, rows, cols, std):
        return (qt, M.quantize(qt, rng.normal(0, std, rows * cols).astype(np.float32)), rows, cols)

    layers = []
    for _ in range(n_layers):
        moe = dict(d=d, f=f, ne=ne, k=k, router=rng.normal(0, 0.1, ne * d).astype(np.float32),
                   qtypes=(O.Q4_K,) * 3, packed=1,
                   gate=q(O.Q4_K, ne * f, d, 0.05)[1], up=q(O.Q4_K, ne * f, d, 0.05)[1],
                   down=q(O.Q4_K, ne * d, f, 0.05)[1])
        layers.append(dict(attn_norm=rng.uniform(0.8, 1.2, d).astype(np.float32),
                           ffn_norm=rng.uniform(0.8, 1.2, d).astype(np.float32),
                           wq=q(O.Q4_K, nh * hd, d, 0.06), wk=q(O.Q4_K, nkv * hd, d, 0.06),
                           wv=q(O.Q4_K, nkv * hd, d, 0.06), wo=q(O.Q4_K, d, nh * hd, 0.06), moe=moe))
    out = q(O.Q6_K, vocab, d, 0.05)
    onorm = rng.uniform(0.8, 1.2, d).astype(np.float32)
    embd = rng.normal(0, 1, (vocab, d)).astype(np.float32)
    return layers, out, onorm, embd, (nh, nkv, hd)


@pytest.fixture(scope="module")
def weights():
    return tiny_model(5)


def test_a_batch_computes_what_each_sequence_would_alone(weights):
    layers, out, onorm, embd, (nh, nkv, hd) = weights
    both = ModelOracle(layers, out, onorm, embd, nh, nkv, hd)
    one = ModelOracle(layers, out, onorm, embd, nh, nkv, hd)
    rng = np.random.default_rng(9)
    for step in range(3):
        toks = rng.integers(0, embd.shape[0], 2)
        nb, lb = both.decode_step([0, 1], toks)
        for i in range(2):
            ni, li = one.decode_step([i], toks[i:i + 1])
            assert ni[0] == nb[i] and np.array_equal(li[0], lb[i]), f"step {step}, sequence {i}"


def test_zero_blocks_reduce_to_embedding_norm_and_head(weights):
    # with every projection and expert zero the layers add nothing: logits = head(norm(embd))
    layers, out, onorm, embd, (nh, nkv, hd) = weights
    zl = []
    for L in layers:
        Z = dict(L)
        for name in ("wq", "wk", "wv", "wo"):
            qt, raw, r, c = L[name]
            Z[name] = (qt, np.zeros_like(raw), r, c)
        Z["moe"] = dict(L["moe"], gate=np.zeros_like(L["moe"]["gate"]), up=np.zeros_like(L["moe"]["up"]),
                        down=np.zeros_like(L["moe"]["down"]))
        zl.append(Z)
    m = ModelOracle(zl, out, onorm, embd, nh, nkv, hd)
    toks = np.array([3, 17], dtype=np.uint32)
    nxt, logits = m.decode_step([0, 1], toks)
    qt, raw, vocab, d = out
    hidden = np.stack([norm(embd[t], onorm, 1e-5) for t in toks])
    want = O.matmul(qt, raw, vocab, d, hidden, 2).reshape(2, vocab)
    assert np.array_equal(logits, want)
    assert [greedy(r) for r in want] == list(nxt)


def test_refusals(weights):
    layers, out, onorm, embd, (nh, nkv, hd) = weights
    m = ModelOracle(layers, out, onorm, embd, nh, nkv, hd)
    with pytest.raises(ValueError):
        m.decode_step([0, 0], [1, 2])
    with pytest.raises(ValueError):
        m.decode_step([0], [embd.shape[0]])


def test_engine_oracle_seeds_are_the_references():
    """The synthetic-engine oracle's layer 0 is ModelWeights::synthesize's (weights/mod.rs:
    43-87): the per-tensor seeds, bound(d) = 1/sqrt(d), and the experts whose synthesis the
    reference's models/l2_cache files pin."""
    from oracle import model as OM
    orc = OM.synthetic_engine(1, 128, 4, 4, 32, 256, 8, 2, 260)
    b = O.lib().or_bound(128)
    L = orc.layers[0]
    assert np.array_equal(L["wq"][1].view(np.float32), O.seeded(0x6761_7275_6461_0002, 128 * 128, b))
    assert np.array_equal(L["moe"]["router"], O.seeded(0x6761_7275_6461_0006, 8 * 128, b))
    assert np.array_equal(orc.table.reshape(-1), O.seeded(0x6761_7275_6461_0001, 260 * 128, b))
    g3 = L["moe"]["gate"].view(np.float32).reshape(8, -1)[3]
    assert np.array_equal(g3, O.synthesize_expert(3)[0])
