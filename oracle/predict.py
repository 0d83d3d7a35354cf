"""CPU restatement of the reference's expert predictor.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the library's predictor
(garuda_amd/csrc/gmoe_predict.cpp). The product never loads it.

Follows ExpertPredictor (garuda/src/predictor/mod.rs:15-134): observe :70-82 (every
prev -> next pair, ids < n only, saturating u32), predict :88-115 (scores summed over
the current ids, zero scores dropped, sort by score descending then id ascending,
truncate to k), score :118-134. Pinned by the reference's own tests (:140-205),
restated in tests/test_predict.py, and by brute force on tiny tables.
"""
from __future__ import annotations

U32_MAX = (1 << 32) - 1


class Predictor:
    def __init__(self, n_experts: int):
        self.n = max(1, n_experts)
        self.counts = [[0] * self.n for _ in range(self.n)]
        self.correct = self.wasted = self.missed = 0

    def observe(self, prev, nxt):
        for p in prev:
            for q in nxt:
                if p < self.n and q < self.n:
                    self.counts[p][q] = min(U32_MAX, self.counts[p][q] + 1)

    def predict(self, current, k):
        if not current or k == 0:
            return []
        score = [0] * self.n
        for p in current:
            if p >= self.n:
                continue
            for q in range(self.n):
                score[q] += self.counts[p][q]
        ranked = [(i, s) for i, s in enumerate(score) if s > 0]
        ranked.sort(key=lambda t: (-t[1], t[0]))
        return [i for i, _ in ranked[:k]]

    def score(self, predicted, actual):
        for p in predicted:
            if p in actual:
                self.correct += 1
            else:
                self.wasted += 1
        for a in actual:
            if a not in predicted:
                self.missed += 1
