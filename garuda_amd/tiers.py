"""The synthetic engine's expert tiers and shared weights, over libgaruda_moe's gmoe_l2_* and
gmoe_fill_seeded (include/garuda_moe.h).

Mirrors garuda's MemoryManager below L1 (garuda/src/memory/mod.rs:114-184) and
weights::ModelWeights::synthesize (weights/mod.rs:43-87): an ExpertTier reads the
`expert_{id}.bin` files of an L2 directory, else of an L3 directory (promoting them into
L2), synthesising and writing the missing ones, and a layer registered from it stages
those experts into the HBM slab (the L1 tier).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from ._lib import GmoeL2Counts, GmoeLayerDesc, lib
from .moe import COMBINE_RANK_ORDER, GATING_MIXTRAL, MoeLayer, _check, _fp

# MemoryTier below L1 (memory/mod.rs:17-24)
TIER_L2, TIER_L3, TIER_SYNTHESISED = 1, 2, 3

# weights/mod.rs:43-51: per-tensor seeds ("garuda" + tag)
SEED_EMBED = 0x6761_7275_6461_0001
SEED_WQ = 0x6761_7275_6461_0002
SEED_WK = 0x6761_7275_6461_0003
SEED_WV = 0x6761_7275_6461_0004
SEED_WO = 0x6761_7275_6461_0005
SEED_ROUTER = 0x6761_7275_6461_0006


def bound(fan_in: int) -> float:
    """weights::bound (weights/mod.rs:38-40): 1 / sqrt(fan_in) in f32."""
    return float(np.float32(1.0) / np.sqrt(np.float32(fan_in)))


def fill_seeded(seed: int, n: int, b: float) -> np.ndarray:
    """weights::seeded (weights/mod.rs:26-35): n uniform values in [-b, b]."""
    out = np.empty(n, dtype=np.float32)
    _check(lib().gmoe_fill_seeded(seed, n, b, _fp(out)))
    return out


def engine_weights(d_model: int, n_experts: int, vocab: int) -> dict:
    """ModelWeights::synthesize (weights/mod.rs:70-87) for these dims: embedding
    [vocab x d], wq/wk/wv/wo [d x d], router [n_experts x d]."""
    d, b = d_model, bound(d_model)
    return dict(embedding=fill_seeded(SEED_EMBED, vocab * d, b).reshape(vocab, d),
                wq=fill_seeded(SEED_WQ, d * d, b), wk=fill_seeded(SEED_WK, d * d, b),
                wv=fill_seeded(SEED_WV, d * d, b), wo=fill_seeded(SEED_WO, d * d, b),
                router=fill_seeded(SEED_ROUTER, n_experts * d, b))


class ExpertTier:
    """The experts id_base .. id_base + n_experts - 1 of an L2 directory.

    lazy=False (gmoe_l2_open): every expert is loaded at open and held; lazy=True
    (gmoe_tiers_open, MemoryManager::new with `l3` as the optional L3 directory): nothing is
    loaded until an expert is fetched, each fetch being one load_uncached."""

    def __init__(self, directory: str | os.PathLike, d_model: int, d_ff: int, n_experts: int, id_base: int = 0,
                 l3: str | os.PathLike | None = None, lazy: bool = False):
        self.d, self.f, self.ne, self.id_base = d_model, d_ff, n_experts, id_base
        self.lazy = lazy or l3 is not None
        h = C.c_void_p()
        if self.lazy:
            _check(lib().gmoe_tiers_open(os.fsencode(directory), os.fsencode(l3) if l3 is not None else None,
                                         d_model, d_ff, n_experts, id_base, C.byref(h)))
        else:
            _check(lib().gmoe_l2_open(os.fsencode(directory), d_model, d_ff, n_experts, id_base, C.byref(h)))
        self._h = h

    @property
    def handle(self):
        if self._h is None:
            raise ValueError("expert tier is closed")
        return self._h

    def counts(self) -> GmoeL2Counts:
        out = GmoeL2Counts()
        _check(lib().gmoe_l2_get_counts(self.handle, C.byref(out)))
        return out

    def locate(self, e: int) -> int:
        """MemoryManager::locate below L1 (memory/mod.rs:99-111): TIER_L2, TIER_L3 or
        TIER_SYNTHESISED."""
        return lib().gmoe_l2_locate(self.handle, e)

    def fetch(self, e: int):
        """One load_uncached of expert e: its (gate [f x d], up [f x d], down [d x f]) as
        copies."""
        ptrs = (C.c_void_p * 3)()
        _check(lib().gmoe_l2_fetch(self.handle, e, ptrs))
        shapes = ((self.f, self.d), (self.f, self.d), (self.d, self.f))
        return tuple(np.ctypeslib.as_array(C.cast(ptrs[p], C.POINTER(C.c_float)), shape=shapes[p]).copy()
                     for p in range(3))

    def layer(self, dev, router: np.ndarray, top_k: int, gating: int = GATING_MIXTRAL,
              combine: int = COMBINE_RANK_ORDER) -> MoeLayer:
        """Register the tier's experts as one MoE layer on `dev`, as MoeEngine runs them:
        the Router's gating (moe/mod.rs:98-100), rank-order combine (:104-109), f32
        products (:82-90). A lazy tier's layer fetches each expert when it is first staged
        (gmoe_l2_layer_register); an eager one is registered from the held weights
        (gmoe_l2_layer_desc). The tier must outlive the layer."""
        router = np.ascontiguousarray(router, dtype=np.float32).reshape(self.ne, self.d)
        lid = C.c_uint32()
        if self.lazy:
            _check(lib().gmoe_l2_layer_register(dev.handle, self.handle, _fp(router), top_k, gating, combine,
                                                C.byref(lid)))
        else:
            desc = GmoeLayerDesc()
            _check(lib().gmoe_l2_layer_desc(self.handle, _fp(router), top_k, gating, combine, C.byref(desc)))
            _check(lib().gmoe_layer_register(dev.handle, C.byref(desc), C.byref(lid)))
        self_ = MoeLayer.__new__(MoeLayer)
        self_.dev = dev
        self_.d, self_.f, self_.ne, self_.k = self.d, self.f, self.ne, top_k
        self_.router = router
        self_._keep = [self, router]
        self_.id = lid.value
        return self_

    def close(self) -> None:
        if self._h is not None:
            lib().gmoe_l2_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()
