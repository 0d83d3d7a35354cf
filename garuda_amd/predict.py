"""Expert prediction and prefetch into the HBM slab: the reference's `ExpertPredictor`
(garuda/src/predictor/mod.rs:15-134) and `PrefetchEngine::observe_step`
(garuda/src/prefetch/mod.rs:77-106), backed by the library (gmoe_predictor_*,
gmoe_prefetch_step).

Expert ids are global, `layer * n_experts + expert`, as the reference's llama backend
feeds them (llama/mod.rs:951-962). A prediction never changes an output: a wrong guess
costs one staged expert, and the forward stages what it needs regardless.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import GmoePredictStats, lib
from .moe import _check


def _ids(a):
    a = np.ascontiguousarray(np.asarray(a, dtype=np.uint32).reshape(-1))
    return a, a.ctypes.data_as(C.POINTER(C.c_uint32)), a.size


@dataclass(frozen=True)
class PredictStats:
    """predictor/mod.rs:22-54"""

    correct: int
    wasted: int
    missed: int

    def precision(self) -> float:
        t = self.correct + self.wasted
        return 0.0 if t == 0 else self.correct / t

    def recall(self) -> float:
        t = self.correct + self.missed
        return 0.0 if t == 0 else self.correct / t


class ExpertPredictor:
    """First-order Markov model over expert usage (predictor/mod.rs:15-134)."""

    def __init__(self, n_experts: int):
        h = C.c_void_p()
        _check(lib().gmoe_predictor_create(n_experts, C.byref(h)))
        self._h = h
        self._n = max(1, n_experts)

    @property
    def handle(self):
        return self._h

    def n_experts(self) -> int:
        return self._n

    def observe(self, prev, nxt) -> None:
        pa, pp, pn = _ids(prev)
        na, npp, nn = _ids(nxt)
        _check(lib().gmoe_predictor_observe(self._h, pp, pn, npp, nn))

    def predict(self, current, k: int) -> list:
        ca, cp, cn = _ids(current)
        out = np.empty(max(k, 1), dtype=np.uint32)
        n = C.c_uint32()
        _check(lib().gmoe_predictor_predict(self._h, cp, cn, k, out.ctypes.data_as(C.POINTER(C.c_uint32)),
                                            C.byref(n)))
        return [int(x) for x in out[:n.value]]

    def score(self, predicted, actual) -> None:
        pa, pp, pn = _ids(predicted)
        aa, ap, an = _ids(actual)
        _check(lib().gmoe_predictor_score(self._h, pp, pn, ap, an))

    def stats(self) -> PredictStats:
        s = GmoePredictStats()
        _check(lib().gmoe_predictor_stats(self._h, C.byref(s)))
        return PredictStats(s.correct, s.wasted, s.missed)

    def counts(self) -> np.ndarray:
        out = np.empty(self._n * self._n, dtype=np.uint32)
        _check(lib().gmoe_predictor_get_counts(self._h, out.ctypes.data_as(C.POINTER(C.c_uint32)), out.size))
        return out.reshape(self._n, self._n)

    def set_counts(self, counts) -> None:
        a = np.ascontiguousarray(counts, dtype=np.uint32).reshape(-1)
        _check(lib().gmoe_predictor_set_counts(self._h, a.ctypes.data_as(C.POINTER(C.c_uint32)), a.size))

    def close(self) -> None:
        if self._h is not None:
            lib().gmoe_predictor_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class PrefetchEngine:
    """PrefetchEngine (prefetch/mod.rs:19-106) over the HBM slab: after a step's forward is
    queued, `observe_step` scores the last prediction, learns the transition, predicts
    the next step's experts and stages the ones of that layer that are not resident.

    Off unless `enabled` is passed as True. The reference's loader warms an expert by
    touching its mmapped pages; here a warm is a host-to-device copy of the whole expert
    (99 MB at the C2 shape), and on a drifting batch-1 decode stream with 6 of 8 experts
    resident the predictions were mostly experts already resident while the rest cost
    copies that saved no miss (0.51 ms a step without, 0.56 with, 23 misses either way)."""

    def __init__(self, dev, predictor: ExpertPredictor, enabled: bool = False, depth: int = 2):
        self.dev, self.predictor, self.enabled, self.depth = dev, predictor, enabled, depth
        self.launched = 0
        self.skipped = 0

    def observe_step(self, layer, id_base: int, previous, used, predicted_last_step) -> list:
        if not self.enabled:
            return []
        pa, pp, pn = _ids(previous)
        ua, up, un = _ids(used)
        la, lp, ln = _ids(predicted_last_step)
        out = np.empty(max(self.depth, 1), dtype=np.uint32)
        n, launched, skipped = C.c_uint32(), C.c_uint32(), C.c_uint32()
        _check(lib().gmoe_prefetch_step(self.dev.handle, self.predictor.handle, layer.id, id_base, pp, pn, up, un,
                                        lp, ln, self.depth, out.ctypes.data_as(C.POINTER(C.c_uint32)),
                                        C.byref(n), C.byref(launched), C.byref(skipped)))
        self.launched += launched.value
        self.skipped += skipped.value
        return [int(x) for x in out[:n.value]]

    def predictor_stats(self) -> PredictStats:
        return self.predictor.stats()
