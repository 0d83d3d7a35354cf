"""The decode step at BASELINE configuration 5's real dimensions, teacher-forced layer by
layer against the oracle: 2 Mixtral-shape layers (d 4096, GQA 32 query / 8 kv heads of 128,
8 experts top-2 of 14336, Q3_K gate/up, Q4_K down and attention projections), a Q6_K head
of 32000 rows, a Q6_K token table kept packed, rope theta 1e6, 8 sequences.

Each step's activations come back from the device (gmoe_model_decode_trace) and every piece
of every layer is restated on the device's own inputs (layer_batch_over, llama/mod.rs:
851-893): the norms, the q/k/v and output projections (quant::matmul), attention over a
restated KV cache holding the device's own k and v (attend_one, :766-821), the residual adds
bit for bit, the MoE layer (feed_forward_batch, :903-1020) and the head, each within the
layer bar (rtol 1e-3, atol 1e-4 of the values' size). The embedding rows are the packed
table's rows dequantised, bit for bit. Four steps: every layer's attention reads the keys
and values the earlier steps appended."""
from __future__ import annotations

import os

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import moe as M
from garuda_amd.attention import KvCache
from oracle import oracle as O
from oracle.attention import KvOracle
from oracle.model import ModelOracle, norm
from tests.test_gpu_model import close, same_bits
from tests.test_gpu_parity import say

pytestmark = pytest.mark.gpu

D, F, NE, K, NH, NKV, HD, VOCAB, NL, NSEQ = 4096, 14336, 8, 2, 32, 8, 128, 32000, 2, 8
THREADS = min(16, len(os.sched_getaffinity(0)))


def c5_weights(seed):
    def g(sd, n, std):
        return M.fill_gaussian(sd, n, 0.0, std, THREADS)

    def q(qt, rows, cols, sd, std=0.02):
        return M.quantize(qt, g(sd, rows * cols, std), THREADS)

    ex = {"gate": q(G.Q3_K, NE * F, D, seed), "up": q(G.Q3_K, NE * F, D, seed + 1), "down": q(G.Q4_K, NE * D, F, seed + 2)}
    layers = []
    for l in range(NL):
        s = seed + 16 * (l + 1)
        moe = dict(d=D, f=F, ne=NE, k=K, router=g(s, NE * D, 0.02), qtypes=(O.Q3_K, O.Q3_K, O.Q4_K), packed=1, **ex)
        layers.append(dict(attn_norm=g(s + 1, D, 0.05) + np.float32(1.0), ffn_norm=g(s + 2, D, 0.05) + np.float32(1.0),
                           wq=(O.Q4_K, q(G.Q4_K, NH * HD, D, s + 3), NH * HD, D),
                           wk=(O.Q4_K, q(G.Q4_K, NKV * HD, D, s + 4), NKV * HD, D),
                           wv=(O.Q4_K, q(G.Q4_K, NKV * HD, D, s + 5), NKV * HD, D),
                           wo=(O.Q4_K, q(G.Q4_K, D, NH * HD, s + 6), D, NH * HD), moe=moe))
    head = (O.Q6_K, q(G.Q6_K, VOCAB, D, seed + 100), VOCAB, D)
    onorm = g(seed + 101, D, 0.05) + np.float32(1.0)
    embd_raw = q(G.Q6_K, VOCAB, D, seed + 102, 1.0)
    return layers, head, onorm, embd_raw


def test_c5_shape_decode_teacher_forced():
    layers, head, onorm, embd_raw = c5_weights(0x6335)
    table = O.dequantize(O.Q6_K, embd_raw, VOCAB * D).reshape(VOCAB, D)
    per_expert = sum(M.byte_size(qt, r * c) for qt, r, c in ((G.Q3_K, F, D), (G.Q3_K, F, D), (G.Q4_K, D, F)))
    with G.Device(0, slab_bytes=NL * NE * (per_expert + 4096) + (256 << 20)) as dev:
        kv = KvCache(dev, NL, NH, NKV, HD, block_size=16, max_positions=64, max_seqs=NSEQ, rope_theta=1e6)
        moe = [G.MoeLayer(dev, D, F, NE, K, L["moe"]["router"], L["moe"]["gate"], L["moe"]["up"], L["moe"]["down"],
                          (G.Q3_K, G.Q3_K, G.Q4_K)) for L in layers]
        dense = {n: [G.DenseWeight(dev, L[n][0], L[n][2], L[n][3], L[n][1]) for L in layers]
                 for n in ("wq", "wk", "wv", "wo")}
        out = G.DenseWeight(dev, head[0], head[2], head[3], head[1])
        model = G.DecodeModel(dev, kv, moe, dense["wq"], dense["wk"], dense["wv"], dense["wo"], out,
                              np.stack([L["attn_norm"] for L in layers]), np.stack([L["ffn_norm"] for L in layers]),
                              onorm, (G.Q6_K, embd_raw, VOCAB, D))
        orc = ModelOracle(layers, head, onorm, table, NH, NKV, HD, max_positions=64, rope_theta=1e6, threads=THREADS,
                          packed=True)
        kvo = KvOracle(NL, NH, NKV, HD, max_positions=64, rope_theta=1e6)
        try:
            seqs = [kv.open_seq() for _ in range(NSEQ)]
            toks = np.random.default_rng(7).integers(0, VOCAB, NSEQ).astype(np.uint32)
            for step in range(4):
                say(f"C5-shape teacher-forced decode step {step}")
                gn, gl, tr, fin = model.decode_step_trace(seqs, toks)
                for l, L in enumerate(orc.layers):
                    T, at = tr[l], f"step {step} layer {l}"
                    x_in = table[toks] if l == 0 else (tr[l - 1]["x_mid"] + tr[l - 1]["moe_out"]).astype(np.float32)
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
                    y, ids, _ = O.feed_forward_batch(L["moe"], T["h_ffn"], threads=THREADS)
                    say(f"  {at}: experts {np.bincount(ids.reshape(-1), minlength=NE).tolist()}")
                    close(f"{at}: MoE layer", T["moe_out"], y)
                same_bits(f"step {step}: final residual", fin["x"],
                          (tr[-1]["x_mid"] + tr[-1]["moe_out"]).astype(np.float32))
                close(f"step {step}: output norm", fin["h"], np.stack([norm(x, onorm, orc.eps) for x in fin["x"]]),
                      rtol=1e-5, atol=1e-6)
                close(f"step {step}: logits", gl, orc._matmul(head, fin["h"]))
                toks = gn
        finally:
            model.close()
            for m in moe:
                m.release()
            for ws in dense.values():
                for w in ws:
                    w.release()
            out.release()
            kv.close()
