"""MoE layers registered straight from GGUF files (MoeLayer.from_gguf over a mapped
checkpoint, gmoe_gguf_layer_desc + gmoe_layer_register) against the oracle computing
the same layer from the same tensor bytes.

Reference behaviour restated: LlamaBackend::from_gguf reads either expert layout
(llama/mod.rs:583-607), and the split and merged layouts give identical outputs
(split_expert_tensors_match_merged_layout, llama/mod.rs:2016-2027).
"""
from __future__ import annotations

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import gguf as gg
from oracle import gguf as OG
from oracle import oracle as O
from tests.test_gpu_parity import ATOL, RTOL, bits, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=1 << 30)
    yield d
    d.close()


def write_model(path, layout, d, f, ne, k, nl, qts, seed):
    rng = np.random.default_rng(seed)
    meta = [("general.architecture", gg.STRING, "llama"), ("llama.embedding_length", gg.U32, d),
            ("llama.feed_forward_length", gg.U32, f), ("llama.block_count", gg.U32, nl),
            ("llama.expert_count", gg.U32, ne), ("llama.expert_used_count", gg.U32, k)]
    tensors = []
    for l in range(nl):
        tensors.append((f"blk.{l}.ffn_gate_inp.weight", [d, ne], G.F32,
                        rng.normal(0, 0.02, (ne, d)).astype(np.float32).tobytes()))
        for (base, rows, cols), qt in zip((("ffn_gate", f, d), ("ffn_up", f, d), ("ffn_down", d, f)), qts):
            raw = G.quantize(qt, rng.normal(0, 0.02, ne * rows * cols).astype(np.float32)).tobytes()
            if layout == "stacked":
                tensors.append((f"blk.{l}.{base}_exps.weight", [cols, rows, ne], qt, raw))
            else:
                per = len(raw) // ne
                tensors += [(f"blk.{l}.{base}.{e}.weight", [cols, rows], qt, raw[e * per:(e + 1) * per])
                            for e in range(ne)]
    path.write_bytes(gg.write_gguf(meta, tensors))
    return path


def oracle_from_file(data: bytes, l: int, math: int):
    """The oracle's layer from the file bytes the oracle's own reader addresses."""
    o = OG.layer(OG.parse(data), len(data), l)
    rt, rs, rn = o["router"]
    router = np.frombuffer(data, np.float32, rn // 4, rs).copy()
    mats = {}
    for name in ("gate", "up", "down"):
        qt, starts, per = o[name]
        mats[name] = np.frombuffer(b"".join(data[s:s + per] for s in starts), dtype=np.uint8).copy()
    qts = tuple(o[n][0] for n in ("gate", "up", "down"))
    return dict(d=o["d"], f=o["f"], ne=o["ne"], k=o["k"], gating=0, combine=0,
                packed=1 if math == G.MATH_PACKED else 0, router=router, qtypes=qts, **mats)


@pytest.mark.parametrize("math", [G.MATH_PACKED, G.MATH_F32])
@pytest.mark.parametrize("qts", [(G.Q4_K,) * 3, (G.Q3_K, G.Q3_K, G.Q4_K), (G.Q6_K, G.Q6_K, G.Q8_0)])
def test_layer_from_gguf_matches_the_oracle(dev, tmp_path, qts, math):
    d, f, ne, k, nl = 256, 512, 8, 2, 2
    outs = {}
    for layout in ("stacked", "split"):
        path = write_model(tmp_path / f"{layout}.gguf", layout, d, f, ne, k, nl, qts, seed=11)
        data = path.read_bytes()
        rng = np.random.default_rng(5)
        with G.Gguf.open(path) as g:
            for l in range(nl):
                say(f"gguf {layout} layer {l} qts={qts} math={math}")
                layer = G.MoeLayer.from_gguf(dev, g, l, math=math)
                try:
                    L = oracle_from_file(data, l, math)
                    for n in (1, 5, 64):
                        hs = rng.normal(0, 1, (n, d)).astype(np.float32)
                        out, ids, w = layer.feed_forward_batch(hs)
                        wout, wids, ww = O.feed_forward_batch(L, hs, None, threads=8)
                        assert np.array_equal(ids, wids), "routing differs"
                        assert np.array_equal(bits(w), bits(ww)), "routing weights differ"
                        assert np.allclose(out, wout, rtol=RTOL, atol=ATOL), f"n={n} max err {np.abs(out - wout).max()}"
                        outs[(layout, l, n)] = out
                finally:
                    layer.release()
    for key, out in outs.items():
        if key[0] == "stacked":
            assert np.array_equal(bits(out), bits(outs[("split",) + key[1:]])), f"layouts differ at {key}"


def test_evicted_experts_restage_from_the_mapping(dev, tmp_path):
    path = write_model(tmp_path / "m.gguf", "stacked", 256, 512, 8, 2, 1, (G.Q4_K,) * 3, seed=3)
    rng = np.random.default_rng(9)
    hs = rng.normal(0, 1, (16, 256)).astype(np.float32)
    with G.Gguf.open(path) as g:
        layer = G.MoeLayer.from_gguf(dev, g, 0)
        try:
            first, ids, _ = layer.feed_forward_batch(hs)
            for e in range(8):
                layer.evict(e)
                assert not layer.is_resident(e)
            again, ids2, _ = layer.feed_forward_batch(hs)  # stages the routed experts again
            assert np.array_equal(ids, ids2) and np.array_equal(bits(first), bits(again))
        finally:
            layer.release()


def test_dense_ffn_layer_from_gguf_is_expert_batch(dev, tmp_path):
    """Ffn::Dense (llama/mod.rs:913-920): `expert_batch` of the one dense expert over every
    token, down(silu(gate h) * up h). A layer without expert tensors comes back from the
    GGUF reader as one expert, top-1, zero router: weight 1, so the combine's y * 1 + 0 is
    the dense arm's output. Checked against the oracle's quant::matmul chain written out
    (packed) or simd::matmul over dequantised weights (f32)."""
    from tests.test_gguf import dense_file
    path = tmp_path / "dense.gguf"
    path.write_bytes(dense_file())
    data = path.read_bytes()
    o = OG.layer(OG.parse(data), len(data), 1)
    d, f = o["d"], o["f"]
    w = {n: (o[n][0], np.frombuffer(data, np.uint8, o[n][2], o[n][1][0]).copy()) for n in ("gate", "up", "down")}
    rng = np.random.default_rng(21)
    with G.Gguf.open(path) as g:
        for math in (G.MATH_PACKED, G.MATH_F32):
            layer = G.MoeLayer.from_gguf(dev, g, 1, math=math)
            try:
                for n in (1, 6, 70):
                    say(f"dense gguf layer math={math} n={n}")
                    hs = rng.normal(0, 1, (n, d)).astype(np.float32)
                    out, ids, wts = layer.feed_forward_batch(hs)
                    assert not ids.any() and np.all(wts == 1.0)
                    if math == G.MATH_PACKED:
                        mm = lambda name, rows, cols, x: O.matmul(w[name][0], w[name][1], rows, cols, x, n, 8)  # noqa: E731
                    else:
                        deq = {k: O.dequantize(v[0], v[1], (f * d)) for k, v in w.items()}
                        mm = lambda name, rows, cols, x: O.simd_matmul(deq[name], rows, cols, x, n, 8)  # noqa: E731
                    gt = mm("gate", f, d, hs)
                    up = mm("up", f, d, hs)
                    h = O.silu(gt) * up
                    want = mm("down", d, f, h).reshape(n, d)
                    assert np.allclose(out, want, rtol=RTOL, atol=ATOL), np.abs(out - want).max()
            finally:
                layer.release()
