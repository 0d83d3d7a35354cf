"""Host-side mirror of Garuda's MoE feed-forward interface, backed by the MI355X library.

The names follow the reference (hanumanit/garuda 0.31.0):
  * `block_layout` / `byte_size` / `dequantize` / `matmul` — quant/mod.rs:41-61,
    :89-98, :104-114, :223-304 (the quant module's public functions);
  * `MoeLayer.feed_forward_batch` — LlamaBackend::feed_forward_batch for Ffn::Moe
    (llama/mod.rs:903-998), returning the output and each token's routed experts;
  * `Device.route` — the gating of llama/mod.rs:938-949 and router::Router::route
    (router/mod.rs:58-118);
  * errors map the C-ABI status codes onto GarudaError's variants (core/mod.rs:10-47).
All arithmetic runs in libgaruda_moe.so on the GPU; nothing here computes results.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import GmoeDenseDesc, GmoeLayerDesc, GmoeSlabStats, GmoeTensor, lib

# ggml type ids, quant/mod.rs:22-30
F32, F16, Q4_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 10, 11, 12, 13, 14
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K",
              Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}
_LAYOUT = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34), Q2_K: (256, 84),
           Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}

GATING_LLAMA, GATING_MIXTRAL, GATING_DEEPSEEK, GATING_QWEN = 0, 1, 2, 3
COMBINE_EXPERT_ORDER, COMBINE_RANK_ORDER = 0, 1
MATH_PACKED, MATH_F32 = 0, 1
LAYOUT_STACKED, LAYOUT_SPLIT = 0, 1
EXPERT_ABSENT, EXPERT_QUEUED, EXPERT_STAGING, EXPERT_RESIDENT = 0, 1, 2, 3


class GarudaError(Exception):
    """Base of the errors the path can return (core/mod.rs:10-47)."""


class ModelError(GarudaError):
    pass


class InferenceError(GarudaError):
    pass


class CacheError(GarudaError):
    pass


class ConfigError(GarudaError):
    pass


class DeviceError(GarudaError):
    pass


class NotFoundError(GarudaError, KeyError):
    """No such GGUF metadata key or tensor (where the reference returns `None`)."""


class InvalidTokenError(GarudaError):
    """A token outside the vocabulary (GarudaError::InvalidToken); `token` is its id."""

    token: int = -1


_STATUS = {1: ModelError, 2: InferenceError, 3: CacheError, 4: ConfigError, 5: DeviceError, 6: NotFoundError,
           7: InvalidTokenError}


def _check(status: int) -> None:
    if status != 0:
        msg = lib().gmoe_last_error().decode(errors="replace")
        err = _STATUS.get(status, GarudaError)(msg)
        if status == 7:
            err.token = int(lib().gmoe_last_invalid_token())
        raise err


def block_layout(qtype: int):
    """(elements per block, bytes per block), or None if unsupported (quant/mod.rs:41-61)."""
    return _LAYOUT.get(qtype)


def byte_size(qtype: int, n: int) -> int:
    """Exact packed size of n elements (quant/mod.rs:89-98)."""
    lay = block_layout(qtype)
    if lay is None:
        raise ModelError(f"tensor type {qtype} is not supported")
    e, b = lay
    if n % e:
        raise ModelError(f"{TYPE_NAMES[qtype]} tensor has {n} elements, not a multiple of the block size {e}")
    return n // e * b


def _fp(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _up(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


def quantize(qtype: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """Build-side quantiser (the reference has none): f32 -> packed GGUF blocks."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(byte_size(qtype, x.size), dtype=np.uint8)
    _check(lib().gmoe_quantize(qtype, _fp(x), x.size, out.ctypes.data, threads))
    return out


def fill_gaussian(seed: int, n: int, mean: float = 0.0, std: float = 1.0, threads: int = 0) -> np.ndarray:
    """n draws of N(mean, std^2), deterministic in seed (splitmix64 + Box-Muller)."""
    out = np.empty(n, dtype=np.float32)
    _check(lib().gmoe_fill_gaussian(seed, mean, std, n, _fp(out), threads))
    return out


# ---- synthetic prefill routing: Zipf-skewed expert loads ----

# Logit offsets, in units of the per-token logit noise, under which top-2 of 8 experts
# picks expert e with the shares of Zipf(s = 1.1): 0.398 0.186 0.119 0.087 0.068 0.055
# 0.047 0.040 (fitted by simulating Gaussian logits; the realised counts of a run are
# what tests and benchmarks report).
ZIPF_MU = (2.134, 1.046, 0.696, 0.469, 0.310, 0.188, 0.084, 0.0)


def skew_direction(seed: int, d: int) -> np.ndarray:
    """A unit vector of R^d, deterministic in seed."""
    u = np.random.default_rng(seed).normal(0.0, 1.0, d)
    return u / np.linalg.norm(u)


def skew_router(router, ne: int, d: int, u, alpha: float = 4.0, wstd: float = 0.02, mu=ZIPF_MU) -> np.ndarray:
    """Router rows with their component along the unit vector u replaced by
    mu[e] * sigma / alpha, sigma = wstd * sqrt(d) being the logit noise of N(0, 1)
    tokens: tokens whose component along u is alpha (skew_tokens) then have logits
    mu[e] * sigma plus noise, so the expert load follows mu. f32 out."""
    R = np.asarray(router, np.float64).reshape(ne, d)
    R = R - np.outer(R @ u, u) + np.outer(np.asarray(mu[:ne], np.float64) * wstd * np.sqrt(d) / alpha, u)
    return R.astype(np.float32).reshape(-1)


def skew_tokens(hs, u, alpha: float = 4.0) -> np.ndarray:
    """N(0, 1) tokens with their component along u set to alpha (a shared mean direction)."""
    H = np.asarray(hs, np.float64)
    return (H + np.outer(alpha - H @ u, u)).astype(np.float32)


@dataclass
class SlabStats:
    hits: int
    misses: int
    evictions: int
    entries: int
    bytes: int
    capacity: int
    h2d_bytes: int


class Device:
    """One MI355X with its HBM expert slab (gmoe_init)."""

    def __init__(self, device: int = 0, slab_bytes: int = 8 << 30):
        h = C.c_void_p()
        _check(lib().gmoe_init(device, slab_bytes, C.byref(h)))
        self._h = h

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if self._h:
            lib().gmoe_shutdown(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # -- single steps of the path --
    def dequantize(self, qtype: int, raw: np.ndarray, n: int) -> np.ndarray:
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        out = np.empty(n, dtype=np.float32)
        _check(lib().gmoe_dequant(self._h, qtype, raw.ctypes.data, raw.size, n, _fp(out)))
        return out

    def matmul(self, qtype: int, w: np.ndarray, rows: int, cols: int, xs: np.ndarray, n: int,
               math: int = MATH_PACKED) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.uint8)
        xs = np.ascontiguousarray(xs, dtype=np.float32).reshape(-1)
        if xs.size != n * cols:
            raise InferenceError(f"matmul dimension mismatch: xs={xs.size}, expected {n * cols}")
        out = np.empty(n * rows, dtype=np.float32)
        _check(lib().gmoe_matmul(self._h, qtype, math, w.ctypes.data, w.size, rows, cols, _fp(xs), n, _fp(out)))
        return out

    def route(self, gating: int, router, x: np.ndarray, ne: int, k: int):
        """Gating of n tokens. router=None means x already holds [n, ne] logits."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.shape[0]
        d = 0 if router is None else x.shape[1]
        ids = np.empty((n, k), dtype=np.uint32)
        w = np.empty((n, k), dtype=np.float32)
        logits = np.empty((n, ne), dtype=np.float32)
        rp = None
        if router is not None:
            router = np.ascontiguousarray(router, dtype=np.float32)
            rp = _fp(router)
        _check(lib().gmoe_route(self._h, gating, rp, _fp(x), d, ne, k, n, _up(ids), _fp(w), _fp(logits)))
        return ids, w, logits

    def dispatch(self, ids: np.ndarray, w: np.ndarray, ne: int):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        n, k = ids.shape
        offsets = np.empty(ne + 1, dtype=np.uint32)
        tok = np.empty(n * k, dtype=np.uint32)
        sw = np.empty(n * k, dtype=np.float32)
        rank = np.empty(n * k, dtype=np.uint32)
        _check(lib().gmoe_dispatch(self._h, _up(ids), _fp(w), n, k, ne, _up(offsets), _up(tok), _fp(sw), _up(rank)))
        return offsets, tok, sw, rank

    def expf(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty_like(x)
        _check(lib().gmoe_expf(self._h, _fp(x), x.size, _fp(y)))
        return y

    def slab_stats(self) -> SlabStats:
        s = GmoeSlabStats()
        _check(lib().gmoe_slab_get_stats(self._h, C.byref(s)))
        return SlabStats(s.hits, s.misses, s.evictions, s.entries, s.bytes, s.capacity, s.h2d_bytes)

    def prefetch_hold(self, hold: bool) -> None:
        """gmoe_prefetch_hold: the staging thread starts nothing new while held."""
        _check(lib().gmoe_prefetch_hold(self._h, 1 if hold else 0))

    def prefetch_wait(self) -> None:
        """gmoe_prefetch_wait: until the staging thread is idle."""
        _check(lib().gmoe_prefetch_wait(self._h))

    def set_kernel_timing(self, on: bool) -> None:
        _check(lib().gmoe_set_kernel_timing(self._h, 1 if on else 0))

    def kernel_time(self, which: int):
        ms, cnt = C.c_double(), C.c_uint64()
        _check(lib().gmoe_kernel_time(self._h, which, C.byref(ms), C.byref(cnt)))
        return ms.value, cnt.value


class MoeLayer:
    """One `Ffn::Moe` layer (llama/mod.rs:501-506) resident on a Device.

    gate/up/down are the packed expert tensors: a stacked uint8 array of
    n_experts*rows rows, or a list of n_experts per-expert arrays (split layout).
    The arrays are borrowed and kept alive by this object, since an evicted expert
    is staged again from them.
    """

    def __init__(self, dev: Device, d_model: int, d_ff: int, n_experts: int, top_k: int,
                 router: np.ndarray, gate, up, down, qtypes, gating: int = GATING_LLAMA,
                 combine: int = COMBINE_EXPERT_ORDER, math: int = MATH_PACKED):
        self.dev = dev
        self.d, self.f, self.ne, self.k = d_model, d_ff, n_experts, top_k
        self._keep = []
        self.router = np.ascontiguousarray(router, dtype=np.float32).reshape(n_experts, d_model)
        self._keep.append(self.router)
        desc = GmoeLayerDesc()
        desc.d_model, desc.d_ff, desc.n_experts, desc.top_k = d_model, d_ff, n_experts, top_k
        desc.gating, desc.combine, desc.math = gating, combine, math
        desc.router = _fp(self.router)
        for name, t, qt in zip(("gate", "up", "down"), (gate, up, down), qtypes):
            desc_t = getattr(desc, name)
            desc_t.qtype = qt
            if isinstance(t, (list, tuple)):
                arrs = [np.ascontiguousarray(a, dtype=np.uint8) for a in t]
                ptrs = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
                self._keep.extend(arrs)
                self._keep.append(ptrs)
                desc_t.layout = LAYOUT_SPLIT
                desc_t.experts = C.cast(ptrs, C.POINTER(C.c_void_p))
            else:
                a = np.ascontiguousarray(t, dtype=np.uint8)
                self._keep.append(a)
                desc_t.layout = LAYOUT_STACKED
                desc_t.data = a.ctypes.data
        lid = C.c_uint32()
        _check(lib().gmoe_layer_register(dev.handle, C.byref(desc), C.byref(lid)))
        self.id = lid.value

    @classmethod
    def from_gguf(cls, dev: Device, gguf, layer: int, gating: int = GATING_LLAMA,
                  combine: int = COMBINE_EXPERT_ORDER, math: int = MATH_PACKED) -> "MoeLayer":
        """Layer `layer` of a GGUF checkpoint (garuda_amd.gguf.Gguf), registered straight
        from the file's bytes: the `Ffn::Moe` arm of LlamaBackend::from_gguf
        (llama/mod.rs:569-607), or for a layer without expert tensors the `Ffn::Dense` arm
        (:608-613) as one expert of weight 1, top-1. The checkpoint stays open while this
        layer lives."""
        desc = GmoeLayerDesc()
        _check(lib().gmoe_gguf_layer_desc(gguf.handle, layer, gating, combine, math, C.byref(desc)))
        self = cls.__new__(cls)
        self.dev = dev
        self.d, self.f, self.ne, self.k = desc.d_model, desc.d_ff, desc.n_experts, desc.top_k
        self._keep = [gguf]
        self.router = np.ctypeslib.as_array(desc.router, shape=(self.ne, self.d)).copy()
        lid = C.c_uint32()
        _check(lib().gmoe_layer_register(dev.handle, C.byref(desc), C.byref(lid)))
        self.id = lid.value
        return self

    def feed_forward_batch(self, hs: np.ndarray, logits: np.ndarray | None = None):
        """(out [n, d], routed ids [n, k], routed weights [n, k]) for n hidden states."""
        hs = np.ascontiguousarray(hs, dtype=np.float32)
        if hs.ndim != 2 or hs.shape[1] != self.d:
            raise InferenceError(f"hidden states must be [n, {self.d}], got {hs.shape}")
        n = hs.shape[0]
        out = np.empty((n, self.d), dtype=np.float32)
        ids = np.empty((n, self.k), dtype=np.uint32)
        w = np.empty((n, self.k), dtype=np.float32)
        if logits is None:
            _check(lib().gmoe_ffn_forward(self.dev.handle, self.id, _fp(hs), n, _fp(out), _up(ids), _fp(w)))
        else:
            logits = np.ascontiguousarray(logits, dtype=np.float32)
            if logits.shape != (n, self.ne):
                raise InferenceError(f"logits must be [{n}, {self.ne}]")
            _check(lib().gmoe_ffn_forward_logits(self.dev.handle, self.id, _fp(hs), _fp(logits), n,
                                                 _fp(out), _up(ids), _fp(w)))
        return out, ids, w

    def forward_async(self, d_hs: int, n: int, d_out: int, d_ids: int = 0, d_w: int = 0,
                      d_logits: int = 0, stream: int = 0) -> None:
        """Device-pointer form (gmoe_ffn_forward_async); pointers are raw addresses."""
        _check(lib().gmoe_ffn_forward_async(self.dev.handle, self.id, d_hs or None, d_logits or None, n,
                                            d_out or None, d_ids or None, d_w or None, stream or None))

    def forward_noalloc(self, d_hs: int, n: int, d_out: int, d_ids: int = 0, d_w: int = 0,
                        d_logits: int = 0, stream: int = 0) -> None:
        """gmoe_ffn_forward_noalloc: as forward_async, with the library's static device
        scratch instead of its arena (no allocation during the call)."""
        _check(lib().gmoe_ffn_forward_noalloc(self.dev.handle, self.id, d_hs or None, d_logits or None, n,
                                              d_out or None, d_ids or None, d_w or None, stream or None))

    def prefetch(self, e: int) -> None:
        _check(lib().gmoe_expert_prefetch(self.dev.handle, self.id, e))

    def is_resident(self, e: int) -> bool:
        return bool(lib().gmoe_expert_is_resident(self.dev.handle, self.id, e))

    def state(self, e: int) -> int:
        """gmoe_expert_state: EXPERT_ABSENT, EXPERT_QUEUED, EXPERT_STAGING or EXPERT_RESIDENT."""
        return int(lib().gmoe_expert_state(self.dev.handle, self.id, e))

    def evict(self, e: int) -> None:
        _check(lib().gmoe_expert_evict(self.dev.handle, self.id, e))

    def release(self) -> None:
        _check(lib().gmoe_layer_release(self.dev.handle, self.id))


class DenseWeight:
    """A dense packed projection on a Device: `Weight::matmul_rows(0, xs, n, out)`
    (llama/mod.rs:148-195) for the attention projections and the output head. `raw` is
    `rows` packed rows of `cols` values of `qtype`; it is copied to the device."""

    MAX_SLICES = 8  # GMOE_DENSE_MAX_SLICES: K slices of forward_slices_async at most

    def __init__(self, dev: Device, qtype: int, rows: int, cols: int, raw, math: int = MATH_PACKED):
        self.dev, self.qtype, self.rows, self.cols, self.math = dev, qtype, rows, cols, math
        a = np.ascontiguousarray(raw, dtype=np.uint8) if not isinstance(raw, (bytes, bytearray, memoryview)) \
            else np.frombuffer(raw, dtype=np.uint8)
        if a.size != byte_size(qtype, rows * cols):
            raise ModelError(f"dense weight: {a.size} bytes for {rows} x {cols} values of type {qtype}")
        desc = GmoeDenseDesc(rows, cols, qtype, math, a.ctypes.data)
        i = C.c_uint32()
        _check(lib().gmoe_dense_register(dev.handle, C.byref(desc), C.byref(i)))
        self.id = i.value

    @classmethod
    def from_gguf(cls, dev: Device, gguf, name: str, math: int = MATH_PACKED) -> "DenseWeight":
        """The tensor `name` of a GGUF checkpoint (ggml dims [cols, rows])."""
        t = gguf.tensor(name)
        if t is None:
            raise ModelError(f"gguf: tensor '{name}' not found")
        cols = t.dims[0]
        rows = t.n_elements() // max(cols, 1)
        return cls(dev, t.ggml_type, rows, cols, t.bytes(), math)

    def matmul_rows(self, xs: np.ndarray) -> np.ndarray:
        """out [n, rows] for xs [n, cols]."""
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        if xs.ndim == 1:
            xs = xs.reshape(1, -1)
        if xs.shape[1] != self.cols:
            raise InferenceError(f"activations must be [n, {self.cols}], got {xs.shape}")
        out = np.empty((xs.shape[0], self.rows), dtype=np.float32)
        _check(lib().gmoe_dense_forward(self.dev.handle, self.id, _fp(xs), xs.shape[0], _fp(out)))
        return out

    def forward_async(self, d_xs: int, n: int, d_out: int, stream: int = 0) -> None:
        _check(lib().gmoe_dense_forward_async(self.dev.handle, self.id, d_xs or None, n, d_out or None,
                                              stream or None))

    def forward_slices_async(self, d_xs: int, n: int, d_parts: int, stream: int = 0) -> int:
        """gmoe_dense_forward_slices_async: the K slices of the output into d_parts
        (MAX_SLICES * n * rows floats), their in-order sum left to the caller; returns the
        slice count."""
        nsl = C.c_uint32(0)
        _check(lib().gmoe_dense_forward_slices_async(self.dev.handle, self.id, d_xs or None, n, d_parts or None,
                                                     C.byref(nsl), stream or None))
        return nsl.value

    def release(self) -> None:
        _check(lib().gmoe_dense_release(self.dev.handle, self.id))
