"""A whole decode step on the GPU (gmoe_model_*, garuda_amd.DecodeModel) against the
oracle's restatement of logits_batch (oracle/model.py): a small model (C1's shape class:
d 256, GQA 8 query heads of 32, 8 experts top-2 of 512; Q4_K projections and experts,
Q6_K head) over three sequences, fed their prompts one token per step and then decoding
greedily, with q, k and v stacked into one projection (2 kv heads: 64-row k and v) and
separate (1 kv head: 32-row k and v).

Under f32 math (Weight::Full) every step's logits match within the layer tolerance, end
to end. Under both maths every layer of every step is also checked teacher-forced: the
step's activations come back from the device (gmoe_model_decode_trace) and each piece of
each layer is restated on the device's own inputs — the norms, the q/k/v and output
projections, attention over a restated KV cache that holds the device's own k and v, the
residual adds (bit for bit) and the MoE layer — each within the layer bar (rtol 1e-3,
atol 1e-4 of the values' size). Fed identical inputs, the int8 quantisation of packed math
rounds identically, so no piece needs a looser bound. (End to end under packed math, a
norm summed in another order can round one int8 value the other way and the KV cache
carries it on; the teacher-forced checks are the parity test there.) Sequences whose
router met a near-tie (the top-k gap below 1e-4) are left out of the end-to-end check.
Refusals leave every sequence where it was."""
from __future__ import annotations

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import moe as M
from garuda_amd.attention import KvCache
from oracle import oracle as O
from oracle.attention import KvOracle
from oracle.model import ModelOracle, norm
from tests.test_gpu_parity import say
from tests.test_model_oracle import tiny_model

pytestmark = pytest.mark.gpu

D, NH, NKV, HD, F, NE, K, VOCAB, NL = 256, 8, 2, 32, 512, 8, 2, 512, 3


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=256 << 20)
    yield d
    d.close()


def gpu_model(dev, w, max_positions=64, max_seqs=4, math=G.MATH_PACKED):
    layers, out, onorm, embd, (nh, nkv, hd) = w
    kv = KvCache(dev, len(layers), nh, nkv, hd, block_size=16, max_positions=max_positions, max_seqs=max_seqs)
    moe, dense = [], {n: [] for n in ("wq", "wk", "wv", "wo")}
    for L in layers:
        m = L["moe"]
        moe.append(G.MoeLayer(dev, m["d"], m["f"], m["ne"], m["k"], m["router"], m["gate"], m["up"], m["down"],
                              m["qtypes"], math=math))
        for n in dense:
            qt, raw, r, c = L[n]
            dense[n].append(G.DenseWeight(dev, qt, r, c, raw, math))
    qt, raw, r, c = out
    head = G.DenseWeight(dev, qt, r, c, raw, math)
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


@pytest.fixture(scope="module", params=[NKV, 1], ids=["qkv-stacked", "qkv-separate"])
def weights(request):
    # 2 kv heads of 32: k and v have 64 rows, whole tiles, and the model stacks q|k|v into
    # one projection; 1 kv head: 32-row k and v, three separate projections
    return tiny_model(11, n_layers=NL, d=D, nh=NH, nkv=request.param, hd=HD, f=F, ne=NE, k=K, vocab=VOCAB)


NEAR_TIE = 1e-4  # router logits this close may rank either way once sums are reordered


def run_steps(dev, weights, math):
    """Per (step, sequence) free of near-ties: (relative max logit error, greedy agrees or
    the top two logits are within 4e-3 of the logits' size)."""
    layers, out, onorm, embd, (nh, nkv, hd) = weights
    parts = gpu_model(dev, weights, math=math)
    model, kv = parts[0], parts[1]
    rows = []
    try:
        orc = ModelOracle(layers, out, onorm, embd, nh, nkv, hd, max_positions=64, packed=math == G.MATH_PACKED)
        seqs = [kv.open_seq() for _ in range(3)]
        prompt = np.random.default_rng(3).integers(0, VOCAB, (3, 6)).astype(np.uint32)
        toks = prompt[:, 0]
        ambiguous = set()
        for step in range(12):  # 6 prompt tokens, then greedy decoding
            say(f"model decode step {step} (math {math})")
            gn, gl = model.decode_step(seqs, toks, want_logits=True)
            on, ol = orc.decode_step(seqs, toks)
            ambiguous |= {i for i, m in enumerate(orc.last_margins) if m < NEAR_TIE}
            for i in range(len(seqs)):
                if i in ambiguous:
                    continue
                scale = float(np.abs(ol[i]).max())
                top = np.sort(ol[i])[-2:]
                rows.append((float(np.abs(gl[i] - ol[i]).max()) / scale,
                             gn[i] == on[i] or top[1] - top[0] <= 4e-3 * scale, step, i))
            toks = prompt[:, step + 1] if step + 1 < prompt.shape[1] else on
        for s in seqs:
            assert all(kv.seq_len(s, l) == 12 for l in range(NL))
    finally:
        release(*parts)
    assert len(rows) >= 24, f"only {len(rows)} (step, sequence) pairs free of near-ties"
    return rows


def test_decode_steps_f32_math(dev, weights):
    for err, same, step, i in run_steps(dev, weights, G.MATH_F32):
        assert err <= 1e-3, f"step {step}, sequence {i}: max error {err:.2e} of the logits' size"
        assert same, f"step {step}, sequence {i}: another greedy token"


def close(what, got, want, rtol=1e-3, atol=1e-4):
    """Within rtol of each value plus atol of the values' size (at least 1)."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    scale = max(1.0, float(np.abs(want).max()))
    err = np.abs(got.astype(np.float64) - want)
    bound = atol * scale + rtol * np.abs(want.astype(np.float64))
    bad = np.flatnonzero(err > bound)
    assert bad.size == 0, (f"{what}: {bad.size} values beyond the bar, worst error {err.max():.3g} "
                           f"(values up to {scale:.3g})")


def same_bits(what, got, want):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{what}: not bit for bit"


@pytest.mark.parametrize("math", [G.MATH_PACKED, G.MATH_F32], ids=["packed", "f32"])
def test_decode_layers_teacher_forced(dev, weights, math):
    layers, out, onorm, embd, (nh, nkv, hd) = weights
    parts = gpu_model(dev, weights, math=math)
    model, kv = parts[0], parts[1]
    orc = ModelOracle(layers, out, onorm, embd, nh, nkv, hd, max_positions=64, packed=math == G.MATH_PACKED)
    kvo = KvOracle(NL, nh, nkv, hd, max_positions=64)  # holds the device's own k and v
    try:
        seqs = [kv.open_seq() for _ in range(3)]
        prompt = np.random.default_rng(4).integers(0, VOCAB, (3, 6)).astype(np.uint32)
        toks = prompt[:, 0]
        for step in range(10):  # 6 prompt tokens, then greedy decoding
            say(f"teacher-forced decode step {step} (math {math})")
            gn, gl, tr, fin = model.decode_step_trace(seqs, toks)
            for l, L in enumerate(orc.layers):
                T, at = tr[l], f"step {step} layer {l}"
                x_in = embd[toks] if l == 0 else (tr[l - 1]["x_mid"] + tr[l - 1]["moe_out"]).astype(np.float32)
                same_bits(f"{at}: residual in", T["x"], x_in)
                close(f"{at}: attention norm", T["h_attn"],
                      np.stack([norm(x, L["attn_norm"], orc.eps) for x in T["x"]]), rtol=1e-5, atol=1e-6)
                for key in ("q", "k", "v"):
                    close(f"{at}: {key}", T[key], orc._matmul(L["w" + key], T["h_attn"]))
                ctx = np.stack([kvo.attend_one(l, s, T["q"][i], T["k"][i], T["v"][i]) for i, s in enumerate(seqs)])
                close(f"{at}: attention", T["context"], ctx)
                close(f"{at}: wo", T["attn_out"], orc._matmul(L["wo"], T["context"]))
                same_bits(f"{at}: attention residual", T["x_mid"], (T["x"] + T["attn_out"]).astype(np.float32))
                close(f"{at}: ffn norm", T["h_ffn"],
                      np.stack([norm(x, L["ffn_norm"], orc.eps) for x in T["x_mid"]]), rtol=1e-5, atol=1e-6)
                y, _, _ = O.feed_forward_batch(L["moe"], T["h_ffn"], threads=8)
                close(f"{at}: MoE layer", T["moe_out"], y)
            same_bits(f"step {step}: final residual", fin["x"],
                      (tr[-1]["x_mid"] + tr[-1]["moe_out"]).astype(np.float32))
            close(f"step {step}: output norm", fin["h"], np.stack([norm(x, onorm, orc.eps) for x in fin["x"]]),
                  rtol=1e-5, atol=1e-6)
            close(f"step {step}: logits", gl, orc._matmul(out, fin["h"]))
            toks = prompt[:, step + 1] if step + 1 < prompt.shape[1] else gn
    finally:
        release(*parts)


def test_graph_steps_equal_eager_steps(dev, weights):
    """Decode steps replayed from the captured graph (the default) against the same steps
    issued launch by launch, on two models of the same weights: next tokens and logits
    bit for bit at every step. The batch goes 3, 2, 3 (a graph per batch size, the second
    3-graph recaptured or kept), positions cross page boundaries (pages of 16), and every
    replay follows the other model's eager work and a synchronisation."""
    a, b = gpu_model(dev, weights), gpu_model(dev, weights)
    ma, kva, mb, kvb = a[0], a[1], b[0], b[1]
    try:
        ma.set_graphs(False)
        sa = [kva.open_seq() for _ in range(3)]
        sb = [kvb.open_seq() for _ in range(3)]
        rng = np.random.default_rng(5)
        toks = rng.integers(0, VOCAB, 3).astype(np.uint32)
        replays = 0
        for step in range(40):
            live = [0, 1, 2] if step < 12 or step >= 20 else [0, 2]
            say(f"graph step {step}, batch {len(live)}")
            ready = mb.graph_ready(len(live))
            na, la = ma.decode_step([sa[i] for i in live], toks[live], want_logits=True)
            nb, lb = mb.decode_step([sb[i] for i in live], toks[live], want_logits=True)
            replays += ready
            assert np.array_equal(na, nb), f"step {step}: next tokens differ"
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), f"step {step}: logits differ"
            toks[live] = na
        assert mb.graph_ready(3) and replays >= 30, f"{replays} steps replayed from a graph"
        for i in range(3):
            assert kva.seq_len(sa[i], NL - 1) == kvb.seq_len(sb[i], NL - 1)
    finally:
        release(*a)
        release(*b)


def test_graph_steps_equal_eager_steps_wide_router(dev):
    """The same comparison on a model of 72 experts, past the speculative front end's 64:
    its graph steps run the FFN's add-norm as a launch of its own (the output projection's
    K slices added there) and the wide front end, and must still match the eager steps
    (reduced output projection, separate add-norm) bit for bit."""
    w = tiny_model(13, n_layers=2, d=D, nh=NH, nkv=NKV, hd=HD, f=F, ne=72, k=K, vocab=VOCAB)
    a, b = gpu_model(dev, w), gpu_model(dev, w)
    ma, kva, mb, kvb = a[0], a[1], b[0], b[1]
    try:
        ma.set_graphs(False)
        sa = [kva.open_seq() for _ in range(3)]
        sb = [kvb.open_seq() for _ in range(3)]
        toks = np.random.default_rng(7).integers(0, VOCAB, 3).astype(np.uint32)
        replays = 0
        for step in range(10):
            say(f"wide-router graph step {step}")
            replays += mb.graph_ready(3)
            na, la = ma.decode_step(sa, toks, want_logits=True)
            nb, lb = mb.decode_step(sb, toks, want_logits=True)
            assert np.array_equal(na, nb), f"step {step}: next tokens differ"
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), f"step {step}: logits differ"
            toks = na
        assert replays >= 8, f"{replays} steps replayed from a graph"
    finally:
        release(*a)
        release(*b)


def test_refusals_leave_the_sequences_unchanged(dev, weights):
    parts = gpu_model(dev, weights, max_positions=3)
    model, kv, moe = parts[0], parts[1], parts[2]
    try:
        a, b = kv.open_seq(), kv.open_seq()
        model.decode_step([a, b], [1, 2])
        with pytest.raises(G.InvalidTokenError) as bad:
            model.decode_step([a, b], [1, VOCAB])
        assert bad.value.token == VOCAB  # the Token GarudaError::InvalidToken carries
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
        # a model wider than a norm workgroup holds (8192) is refused at create
        wide = 8196
        with pytest.raises(G.ConfigError):
            G.DecodeModel(dev, kv, moe, *[parts[3][n] for n in ("wq", "wk", "wv", "wo")], parts[4],
                          np.ones((NL, wide), np.float32), np.ones((NL, wide), np.float32), np.ones(wide, np.float32),
                          np.zeros((VOCAB, wide), np.float32))
    finally:
        release(*parts)


def test_failed_graph_step_leaves_the_sequences_unchanged(dev, weights):
    """A graph-replayed step plans every layer's positions, reserves the attention scratch
    they need and only then commits them; a step that fails after committing gives them
    back. With the reservation refused (a test hook standing in for an allocation failure)
    the step is an error and every sequence keeps its length and the pool its free pages;
    the next steps then match a model that never failed, bit for bit."""
    a, b = gpu_model(dev, weights, max_positions=256), gpu_model(dev, weights, max_positions=256)
    ma, kva, mb, kvb = a[0], a[1], b[0], b[1]
    try:
        sa = [kva.open_seq() for _ in range(2)]
        sb = [kvb.open_seq() for _ in range(2)]
        toks = np.array([5, 9], np.uint32)
        for step in range(3):
            na = ma.decode_step(sa, toks)
            nb = mb.decode_step(sb, toks)
            assert np.array_equal(na, nb)
            toks = na
        # a batch size of a new graph: its scratch is reserved before anything commits
        lens = [kva.seq_len(s, l) for s in sa for l in range(NL)]
        free = kva.free_pages()
        kva.fail_reserves(1)
        with pytest.raises(G.DeviceError):
            ma.decode_step(sa[:1], toks[:1])
        assert [kva.seq_len(s, l) for s in sa for l in range(NL)] == lens
        assert kva.free_pages() == free
        for step in range(66):  # past pages (16 positions) and a chunk bucket (64 positions)
            say(f"after a failed step: step {step}")
            na, la = ma.decode_step(sa, toks, want_logits=True)
            nb, lb = mb.decode_step(sb, toks, want_logits=True)
            assert np.array_equal(na, nb) and np.array_equal(la.view(np.uint32), lb.view(np.uint32)), step
            toks = na
        assert kva.free_pages() == kvb.free_pages()
    finally:
        release(*a)
        release(*b)


def test_graph_cache_serves_drifting_batches_over_a_long_window(dev):
    """Continuous batching: the batch size drifts between 1 and 3 as sequences join and
    leave, over a 32768-position window. Graphs are kept per (batch, chunk bucket) and
    replayed; each replayed step's attention spans the live context's bucket, not the
    window. Every step matches a model issuing every launch, bit for bit."""
    w = tiny_model(17, n_layers=2, d=D, nh=NH, nkv=NKV, hd=HD, f=F, ne=NE, k=K, vocab=VOCAB)
    a, b = gpu_model(dev, w, max_positions=32768), gpu_model(dev, w, max_positions=32768)
    ma, kva, mb, kvb = a[0], a[1], b[0], b[1]
    try:
        ma.set_graphs(False)
        sa = [kva.open_seq() for _ in range(3)]
        sb = [kvb.open_seq() for _ in range(3)]
        rng = np.random.default_rng(5)
        toks = rng.integers(0, VOCAB, 3).astype(np.uint32)
        pattern = [3, 2, 3, 1, 3, 2, 2, 3, 1, 1]
        replays = 0
        for step in range(40):
            n = pattern[step % len(pattern)]
            live = list(range(n))
            replays += mb.graph_ready(n)
            say(f"drifting batch step {step}, n={n}")
            na, la = ma.decode_step([sa[i] for i in live], toks[live], want_logits=True)
            nb, lb = mb.decode_step([sb[i] for i in live], toks[live], want_logits=True)
            assert np.array_equal(na, nb), f"step {step}: next tokens differ"
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), f"step {step}: logits differ"
            toks[live] = na
        assert replays >= 30, f"{replays} steps replayed from a graph"
    finally:
        release(*a)
        release(*b)


def test_model_layers_are_kept_resident_during_a_step(dev, weights):
    """A model step reads every expert of its layers through the device pointer tables,
    so they are held in the slab from the residency check until the step's device work is
    done: an eviction requested meanwhile is refused, and after the step it goes through.
    (Between steps, the staging thread or another call may evict them; the next step then
    refuses cleanly.)"""
    parts = gpu_model(dev, weights)
    model, kv, moe = parts[0], parts[1], parts[2]
    try:
        s = kv.open_seq()
        model.decode_step([s], [1])
        import threading
        errs, done = [], threading.Event()

        import time
        held = [0]

        def evictor():
            while not done.is_set():
                try:
                    moe[0].evict(0)
                    moe[0].prefetch(0)
                    time.sleep(0.002)
                except G.CacheError as e:
                    held[0] += "in use by a model step" in str(e)  # refused while a step held the layer
                except Exception as e:  # noqa: BLE001 - reported below
                    errs.append(e)
                    return

        t = threading.Thread(target=evictor)
        t.start()
        ok = 0
        try:
            for step in range(30):
                try:
                    model.decode_step([s], [step % VOCAB])
                    ok += 1
                except G.CacheError:
                    pass  # the expert was out between steps: refused before any device work
        finally:
            done.set()
            t.join()
        say(f"{ok} of 30 steps ran; {held[0]} evictions refused while a step held the layer")
        assert not errs, errs
        assert ok > 0
    finally:
        release(*parts)


def gpu_model_packed_table(dev, w, embd_qt, math, max_positions=64, tied=True):
    """gpu_model with the token table kept packed (embd_qt rows) and, with tied, the head
    taken from it (llama/mod.rs:565-571); returns the parts and the oracle's f32 table and
    head."""
    layers, out, onorm, embd, (nh, nkv, hd) = w
    vocab, d = embd.shape
    raw = M.quantize(embd_qt, embd.reshape(-1))
    table = O.dequantize(embd_qt, raw, vocab * d).reshape(vocab, d)
    kv = KvCache(dev, len(layers), nh, nkv, hd, block_size=16, max_positions=max_positions, max_seqs=4)
    moe, dense = [], {n: [] for n in ("wq", "wk", "wv", "wo")}
    for L in layers:
        m = L["moe"]
        moe.append(G.MoeLayer(dev, m["d"], m["f"], m["ne"], m["k"], m["router"], m["gate"], m["up"], m["down"],
                              m["qtypes"], math=math))
        for n in dense:
            qt, r, rr, c = L[n]
            dense[n].append(G.DenseWeight(dev, qt, rr, c, r, math))
    qt, r, rr, c = out
    head = None if tied else G.DenseWeight(dev, qt, rr, c, r, math)
    model = G.DecodeModel(dev, kv, moe, dense["wq"], dense["wk"], dense["wv"], dense["wo"], head,
                          np.stack([L["attn_norm"] for L in layers]), np.stack([L["ffn_norm"] for L in layers]),
                          onorm, (embd_qt, raw, vocab, d), output_math=math)
    ohead = (embd_qt, raw, vocab, d) if tied else out
    return (model, kv, moe, dense, head), table, ohead


@pytest.mark.parametrize("embd_qt", [G.Q6_K, G.Q8_0, G.Q4_K, G.Q3_K])
def test_packed_token_table_with_tied_head(dev, weights, embd_qt):
    """token_embd kept packed in HBM (Weight::Packed): each token's row is dequantised on the
    device, bit for bit the reference's dequantize (the first layer's residual input is
    compared bit for bit), and the head tied to the same table (has_tied_embeddings): f32
    math end to end against the oracle's model over the same dequantised table and head."""
    layers, out, onorm, embd, (nh, nkv, hd) = weights
    parts, table, ohead = gpu_model_packed_table(dev, weights, embd_qt, G.MATH_F32)
    model, kv = parts[0], parts[1]
    try:
        orc = ModelOracle(layers, ohead, onorm, table, nh, nkv, hd, max_positions=64, packed=False)
        seqs = [kv.open_seq() for _ in range(2)]
        toks = np.random.default_rng(31).integers(0, VOCAB, 2).astype(np.uint32)
        ambiguous = set()
        for step in range(8):
            say(f"packed token table {embd_qt}, step {step}")
            gn, gl, tr, _ = model.decode_step_trace(seqs, toks)
            same_bits(f"step {step}: embedding rows", tr[0]["x"], table[toks])
            on, ol = orc.decode_step(seqs, toks)
            ambiguous |= {i for i, m in enumerate(orc.last_margins) if m < NEAR_TIE}
            for i in range(2):
                if i in ambiguous:
                    continue
                scale = float(np.abs(ol[i]).max())
                assert float(np.abs(gl[i] - ol[i]).max()) <= 1e-3 * scale, (step, i)
            toks = on
        # graph-replayed steps read the tokens from device memory: same rows
        for step in range(3):
            nxt, lg = model.decode_step(seqs, toks, want_logits=True)
            on, ol = orc.decode_step(seqs, toks)
            for i in range(2):
                if i not in ambiguous:
                    assert float(np.abs(lg[i] - ol[i]).max()) <= 1e-3 * float(np.abs(ol[i]).max())
            toks = on
    finally:
        _release_tied(*parts)


def _release_tied(model, kv, moe, dense, head):
    model.close()
    for m in moe:
        m.release()
    for ws in dense.values():
        for x in ws:
            x.release()
    if head is not None:
        head.release()
    kv.close()


@pytest.fixture(scope="module")
def wide_weights():
    # d 512: the MoE layer, q, o and the head take the MFMA products at prefill sizes
    return tiny_model(23, n_layers=2, d=512, nh=8, nkv=2, hd=64, f=512, ne=8, k=2, vocab=512)


@pytest.mark.parametrize("n_prompt", [70, 300])
def test_prefill_equals_the_prompt_token_by_token(dev, wide_weights, n_prompt):
    """forward_tail (llama/mod.rs:1027-1116): a prompt through the model in chunks of up to
    256 positions, layer-major (the projections and the MoE layer as batched products: the
    MFMA paths at these sizes), against the oracle fed the same prompt one token per step
    (the reference's layer-major and token-major passes are the same arithmetic). f32 math:
    the last positions' logits within 1e-3 of their size, the same greedy tokens where the
    top two are apart; the KV cache the prefill leaves is checked by decoding on from it."""
    weights = wide_weights
    layers, out, onorm, embd, (nh, nkv, hd) = weights
    NL = len(layers)
    VOCAB = embd.shape[0]
    parts = gpu_model(dev, weights, max_positions=320, math=G.MATH_F32)
    model, kv = parts[0], parts[1]
    try:
        orc = ModelOracle(layers, out, onorm, embd, nh, nkv, hd, max_positions=320, packed=False)
        s = kv.open_seq()
        prompt = np.random.default_rng(n_prompt).integers(0, VOCAB, n_prompt).astype(np.uint32)
        say(f"prefill of {n_prompt} tokens")
        gn, gl = model.prefill(s, prompt, n_last=3, want_logits=True)
        assert all(kv.seq_len(s, l) == n_prompt for l in range(NL))
        ol, margins = [], []
        for t in prompt:
            on, lo = orc.decode_step([s], [t])
            ol.append(lo[0])
            margins.append(orc.last_margins[0])
        if min(margins) < NEAR_TIE:
            pytest.skip("the oracle's router met a near-tie in this prompt")
        for j in range(3):
            want = ol[n_prompt - 3 + j]
            scale = float(np.abs(want).max())
            assert float(np.abs(gl[j] - want).max()) <= 1e-3 * scale, j
            top = np.sort(want)[-2:]
            if top[1] - top[0] > 4e-3 * scale:
                assert gn[j] == int(np.argmax(want)), j
        toks = np.array([on[0]], np.uint32)
        for step in range(4):  # decoding on from the prefilled cache
            gnd, gld = model.decode_step([s], toks, want_logits=True)
            on, lo = orc.decode_step([s], toks)
            assert float(np.abs(gld[0] - lo[0]).max()) <= 1e-3 * float(np.abs(lo[0]).max()), step
            toks = np.array([on[0]], np.uint32)
    finally:
        release(*parts)


def test_prefill_refusals_leave_the_sequence_unchanged(dev, weights):
    parts = gpu_model(dev, weights, max_positions=40)
    model, kv = parts[0], parts[1]
    try:
        s = kv.open_seq()
        model.prefill(s, np.arange(10, dtype=np.uint32))
        with pytest.raises(G.InvalidTokenError):
            model.prefill(s, [1, 2, VOCAB])
        with pytest.raises(G.CacheError):  # 10 + 31 positions exceed the window of 40
            model.prefill(s, np.zeros(31, np.uint32))
        with pytest.raises(G.InferenceError):
            model.prefill(s, [1, 2], n_last=3)
        assert all(kv.seq_len(s, l) == 10 for l in range(NL))
        model.prefill(s, np.arange(30, dtype=np.uint32))
        assert kv.seq_len(s, NL - 1) == 40
    finally:
        release(*parts)
