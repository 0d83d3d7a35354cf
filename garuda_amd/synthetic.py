"""garuda's synthetic engine (MoeEngine, garuda/src/moe/mod.rs) on the device, generalised to
several layers and grouped-query heads: BASELINE configuration 1 (4 layers, d 256, 8 query
/ 2 kv heads of 32, 8 experts top-2 of 512, vocab 512).

The reference engine is one block: x = embed(token); x += attention(rmsnorm(x));
x += moe_ffn(rmsnorm(x)); logits = embedding . rmsnorm(x) (moe/mod.rs:115-135, :147-187).
rmsnorm carries no weight (simd/mod.rs:166-173), which is llama's norm with unit weights
exactly, and the head is tied to the embedding, so the engine is the library's decode step
(gmoe_model_*) with unit norm weights and the embedding as an F32 output projection. The
experts come from ExpertTier (the L2 files, synthesised when missing) and run as MoeEngine
runs them: the Router's gating, rank-order combine, f32 products. The shared weights are
weights::ModelWeights::synthesize's (weights/mod.rs:70-87): seeded uniform draws with the
reference's per-tensor seeds. Layer l > 0 (the reference has one block) uses each seed
XOR (l << 32), and its experts are the directory's ids l*n_experts .. (l+1)*n_experts - 1;
with kv heads fewer than query heads, wk and wv have n_kv*head_dim rows.
"""
from __future__ import annotations

import numpy as np

from .attention import KvCache
from .model import DecodeModel
from .moe import COMBINE_RANK_ORDER, F32, GATING_MIXTRAL, MATH_F32, DenseWeight
from .tiers import (SEED_EMBED, SEED_ROUTER, SEED_WK, SEED_WO, SEED_WQ, SEED_WV, ExpertTier, bound,
                    fill_seeded)

NORM_EPS = 1e-5  # moe/mod.rs:24


def layer_seed(seed: int, layer: int) -> int:
    return seed ^ (layer << 32)


class SyntheticEngine:
    """MoeEngine's model on the device. `directory` is the L2 tier (expert_{id}.bin)."""

    def __init__(self, dev, directory, n_layers: int = 4, d_model: int = 256, n_heads: int = 8, n_kv_heads: int = 2,
                 head_dim: int = 32, d_ff: int = 512, n_experts: int = 8, top_k: int = 2, vocab: int = 512,
                 gating: int = GATING_MIXTRAL, max_positions: int = 2048, max_seqs: int = 4, rope_theta: float = 1e4):
        if n_heads * head_dim != d_model:
            raise ValueError("the engine's attention slices d_model into its heads (attention/mod.rs:19-28)")
        self.dims = dict(n_layers=n_layers, d_model=d_model, n_heads=n_heads, n_kv_heads=n_kv_heads,
                         head_dim=head_dim, d_ff=d_ff, n_experts=n_experts, top_k=top_k, vocab=vocab)
        d, kvd, b = d_model, n_kv_heads * head_dim, bound(d_model)
        self.embedding = fill_seeded(SEED_EMBED, vocab * d, b).reshape(vocab, d)
        self.tiers, self.moe, self.dense = [], [], {n: [] for n in ("wq", "wk", "wv", "wo")}
        self.raw = []  # per layer: the shared weights as f32 arrays (for checkers)
        try:
            for l in range(n_layers):
                w = dict(wq=fill_seeded(layer_seed(SEED_WQ, l), d * d, b),
                         wk=fill_seeded(layer_seed(SEED_WK, l), kvd * d, b),
                         wv=fill_seeded(layer_seed(SEED_WV, l), kvd * d, b),
                         wo=fill_seeded(layer_seed(SEED_WO, l), d * d, b),
                         router=fill_seeded(layer_seed(SEED_ROUTER, l), n_experts * d, b))
                self.raw.append(w)
                tier = ExpertTier(directory, d, d_ff, n_experts, id_base=l * n_experts)
                self.tiers.append(tier)
                self.moe.append(tier.layer(dev, w["router"], top_k, gating, COMBINE_RANK_ORDER))
                for name, rows in (("wq", d), ("wk", kvd), ("wv", kvd), ("wo", d)):
                    self.dense[name].append(DenseWeight(dev, F32, rows, d, w[name].view(np.uint8), MATH_F32))
            self.head = DenseWeight(dev, F32, vocab, d, self.embedding.reshape(-1).view(np.uint8), MATH_F32)
            self.kv = KvCache(dev, n_layers, n_heads, n_kv_heads, head_dim, block_size=16,
                              max_positions=max_positions, max_seqs=max_seqs, rope_theta=rope_theta)
            ones = np.ones((n_layers, d), np.float32)
            self.model = DecodeModel(dev, self.kv, self.moe, self.dense["wq"], self.dense["wk"], self.dense["wv"],
                                     self.dense["wo"], self.head, ones, ones, ones[0], self.embedding,
                                     rms_eps=NORM_EPS)
        except Exception:
            self.close()
            raise

    def open_seq(self) -> int:
        return self.kv.open_seq()

    def step(self, seqs, tokens, want_logits: bool = False):
        """One token for each sequence: the greedy next tokens (and the logits)."""
        return self.model.decode_step(seqs, tokens, want_logits)

    def generate(self, prompt, n_new: int):
        """Greedy batch-1 generation: the prompt one token at a time (MoeEngine::hidden
        steps through every unseen token), then n_new tokens."""
        seq = self.open_seq()
        nxt = None
        for t in prompt:
            nxt = self.step([seq], [int(t)])[0]
        out = []
        for _ in range(n_new):
            out.append(int(nxt))
            nxt = self.step([seq], [int(nxt)])[0]
        self.kv.close_seq(seq)
        return out

    def close(self) -> None:
        m = getattr(self, "model", None)
        if m is not None:
            m.close()
        for x in self.moe:
            x.release()
        for ws in self.dense.values():
            for x in ws:
                x.release()
        if getattr(self, "head", None) is not None:
            self.head.release()
        if getattr(self, "kv", None) is not None:
            self.kv.close()
        for t in self.tiers:
            t.close()
        self.moe, self.tiers = [], []
        self.dense = {n: [] for n in self.dense}
        self.head = self.kv = self.model = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()
