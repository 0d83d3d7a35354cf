"""CPU restatement of one decode step of the whole model — TEST INFRASTRUCTURE ONLY
(imported by tests/ as the checker; the product never loads it).

LlamaBackend::logits_batch for its decode case (garuda/src/llama/mod.rs:1134-1206):
every sequence takes one new token.

    x = token_embd.row(token)                                       (:1179-1185)
    per layer (layer_batch_over, :851-893):
        h = norm(x, attn_norm); q, k, v = wq h, wk h, wv h          (:743-757)
        context = attend_one(q, k, v) per token                     (:766-821)
        x += wo context; h = norm(x, ffn_norm); x += ffn(h)
    x = norm(x, output_norm); logits = output x                     (:1191-1199)
    next = the first index of the largest logit                     (runtime/mod.rs:98-105)

norm(x, w) is simd::rmsnorm (simd/mod.rs:166-173: the f32 mean of the squares summed
left to right, scale = 1 / sqrt(mean + eps), x *= scale) then x *= w elementwise
(`mul_assign`). The projections are quant::matmul under packed math (oracle.matmul) or
simd::matmul over the dequantised weights under f32 math, the attention KvOracle
(oracle/attention.py), the MoE layer oracle.feed_forward_batch in the same math.
"""
from __future__ import annotations

import numpy as np

from . import oracle as O
from .attention import KvOracle


def rmsnorm(x: np.ndarray, eps: float) -> np.ndarray:
    """simd::rmsnorm of one row: the squares rounded to f32 and summed in order."""
    x = np.asarray(x, dtype=np.float32)
    if x.size == 0:
        return x.copy()
    sq = (x * x).astype(np.float32)
    mean_sq = np.float32(np.cumsum(sq, dtype=np.float32)[-1] / np.float32(x.size))
    scale = np.float32(np.float32(1.0) / np.sqrt(np.float32(mean_sq + np.float32(eps))))
    return (x * scale).astype(np.float32)


def norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    return (rmsnorm(x, eps) * np.asarray(w, dtype=np.float32)).astype(np.float32)


def greedy(logits: np.ndarray) -> int:
    """runtime::sample at temperature 0: fold from (0, -inf), keeping strict improvements."""
    bi, bv = 0, np.float32(-np.inf)
    for i, v in enumerate(np.asarray(logits, dtype=np.float32)):
        if v > bv:
            bi, bv = i, v
    return bi


class ModelOracle:
    """layers: per layer a dict with attn_norm, ffn_norm, wq/wk/wv/wo as (qtype, raw,
    rows, cols) and moe (an oracle.feed_forward_batch layer dict); output: (qtype, raw,
    vocab, d); output_norm [d]; token_embd [vocab, d] f32."""

    def __init__(self, layers, output, output_norm, token_embd, n_heads, n_kv_heads, head_dim, rms_eps=1e-5,
                 max_positions=2048, rope_theta=10000.0, threads=8, packed=True):
        # packed: Weight::Packed (quant::matmul, int8 activations); else Weight::Full
        # (simd::matmul over the dequantised weights), for the projections and the experts
        self.packed, self._deq = packed, {}
        if not packed:
            layers = [dict(L, moe=dict(L["moe"], packed=0)) for L in layers]
        self.layers, self.output, self.output_norm = layers, output, np.asarray(output_norm, dtype=np.float32)
        self.table = np.asarray(token_embd, dtype=np.float32)
        self.eps, self.threads = rms_eps, threads
        self.kv = KvOracle(len(layers), n_heads, n_kv_heads, head_dim, max_positions=max_positions,
                           rope_theta=rope_theta)
        # per token of the last step, the smallest gap over the layers between the k-th and
        # (k+1)-th largest router logit (in float64): where it is tiny, any reordering of
        # the sums upstream may pick the other expert
        self.last_margins = None

    def _matmul(self, w, xs):
        qt, raw, rows, cols = w
        n = xs.shape[0]
        if self.packed:
            return O.matmul(qt, raw, rows, cols, xs, n, threads=self.threads).reshape(n, rows)
        key = id(raw)
        if key not in self._deq:
            self._deq[key] = (raw, O.dequantize(qt, raw, rows * cols, checked=False).reshape(rows, cols))
        return O.simd_matmul(self._deq[key][1], rows, cols, xs, n, threads=self.threads).reshape(n, rows)

    def decode_step(self, seqs, tokens):
        """(next tokens, logits [n, vocab]) of one step; seqs distinct."""
        n = len(seqs)
        if len(set(seqs)) != n:
            raise ValueError("a sequence appears twice in one decode step")
        vocab = self.table.shape[0]
        for t in tokens:
            if t >= vocab:
                raise ValueError(f"token {t} outside the vocabulary")
        xs = [self.table[t].copy() for t in tokens]
        margins = np.full(n, np.inf)
        for l, L in enumerate(self.layers):
            hs = np.stack([norm(x, L["attn_norm"], self.eps) for x in xs])
            q, k, v = self._matmul(L["wq"], hs), self._matmul(L["wk"], hs), self._matmul(L["wv"], hs)
            ctx = np.stack([self.kv.attend_one(l, s, q[i], k[i], v[i]) for i, s in enumerate(seqs)])
            ao = self._matmul(L["wo"], ctx.astype(np.float32))
            hf = []
            for i in range(n):
                xs[i] = (xs[i] + ao[i]).astype(np.float32)
                hf.append(norm(xs[i], L["ffn_norm"], self.eps))
            mo = L["moe"]
            if mo["k"] < mo["ne"]:
                lg = np.stack(hf).astype(np.float64) @ np.asarray(mo["router"], dtype=np.float64).reshape(mo["ne"], -1).T
                srt = np.sort(lg, axis=1)
                margins = np.minimum(margins, srt[:, -mo["k"]] - srt[:, -mo["k"] - 1])
            ffn, _, _ = O.feed_forward_batch(mo, np.stack(hf), threads=self.threads)
            for i in range(n):
                xs[i] = (xs[i] + ffn[i]).astype(np.float32)
        self.last_margins = margins
        hidden = np.stack([norm(x, self.output_norm, self.eps) for x in xs])
        logits = self._matmul(self.output, hidden)
        return np.array([greedy(r) for r in logits], dtype=np.uint32), logits


# ---- garuda's synthetic engine (MoeEngine, moe/mod.rs:67-187) as a ModelOracle ----

SEED_EMBED, SEED_WQ, SEED_WK, SEED_WV, SEED_WO, SEED_ROUTER = (0x6761_7275_6461_0000 + i for i in range(1, 7))


def engine_layer_seed(seed: int, layer: int) -> int:
    """Layer l's seed for a tensor of the (one-block) reference engine: seed XOR (l << 32)."""
    return seed ^ (layer << 32)


def engine_experts(d, f, ids):
    """Stacked F32 gate, up, down of the synthesised experts `ids` (weights/mod.rs:98-109)."""
    g, u, dn = zip(*(O.synthesize_expert(i, d, f) for i in ids))
    as_u8 = lambda parts: np.concatenate(parts).astype("<f4").view(np.uint8)
    return as_u8(g), as_u8(u), as_u8(dn)


def synthetic_engine(n_layers, d, nh, nkv, hd, f, ne, k, vocab, max_positions=2048, threads=8):
    """MoeEngine generalised to n_layers grouped-query layers, from the oracle's own
    generators: ModelWeights::synthesize's seeded tensors (weights/mod.rs:70-87; layer l's
    seeds XOR (l << 32)), layer l's experts l*ne .. (l+1)*ne - 1, unit norm weights
    (simd::rmsnorm carries none), the Mixtral router with rank-order combine
    (moe/mod.rs:98-109), f32 products, and the head tied to the embedding."""
    b, kvd = O.lib().or_bound(d), nkv * hd
    emb = O.seeded(SEED_EMBED, vocab * d, b).reshape(vocab, d)
    f32 = lambda a, rows, cols: (O.F32, np.ascontiguousarray(a, np.float32).view(np.uint8), rows, cols)
    layers = []
    for l in range(n_layers):
        gate, up, down = engine_experts(d, f, range(l * ne, (l + 1) * ne))
        moe = dict(d=d, f=f, ne=ne, k=k, gating=1, combine=1, packed=0, qtypes=(O.F32,) * 3,
                   router=O.seeded(engine_layer_seed(SEED_ROUTER, l), ne * d, b), gate=gate, up=up, down=down)
        layers.append(dict(attn_norm=np.ones(d, np.float32), ffn_norm=np.ones(d, np.float32),
                           wq=f32(O.seeded(engine_layer_seed(SEED_WQ, l), d * d, b), d, d),
                           wk=f32(O.seeded(engine_layer_seed(SEED_WK, l), kvd * d, b), kvd, d),
                           wv=f32(O.seeded(engine_layer_seed(SEED_WV, l), kvd * d, b), kvd, d),
                           wo=f32(O.seeded(engine_layer_seed(SEED_WO, l), d * d, b), d, d), moe=moe))
    return ModelOracle(layers, f32(emb, vocab, d), np.ones(d, np.float32), emb, nh, nkv, hd, packed=False,
                       max_positions=max_positions, threads=threads)
