"""Dense projections (gmoe_dense_*: Weight::matmul_rows, llama/mod.rs:148-195) against
the oracle's quant::matmul (packed math) and simd::matmul over the dequantised rows (f32
math), at decode and prefill sizes, ragged shapes and the output head's shape.

A row's dot may be split over K and the slices added in order, so the bound is the
summation-order one: |got - want| <= 1e-5 * sum_k |w_k x_k| + 1e-6.
"""
from __future__ import annotations

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import gguf as gg
from oracle import oracle as O
from tests.helpers import fast_random_blocks
from tests.test_gpu_parity import bits, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=256 << 20)
    yield d
    d.close()


def check(dev, qtype, rows, cols, ns, math, seed=0, raw=None):
    e, _ = O.block_layout(qtype)
    if raw is None:
        raw = fast_random_blocks(qtype, rows * cols // e, 31 + qtype + seed)
    W = G.DenseWeight(dev, qtype, rows, cols, raw, math)
    deq = O.dequantize(qtype, raw, rows * cols, checked=False).reshape(rows, cols)
    try:
        for n in ns:
            say(f"dense {qtype} {rows}x{cols} math={math} n={n}")
            xs = np.random.default_rng(seed * 1000 + n).normal(0, 1, (n, cols)).astype(np.float32)
            got = W.matmul_rows(xs)
            if math == G.MATH_PACKED:
                want = O.matmul(qtype, raw, rows, cols, xs, n, threads=8).reshape(n, rows)
            else:
                want = O.simd_matmul(deq, rows, cols, xs, n, threads=8).reshape(n, rows)
            scale = np.abs(xs) @ np.abs(deq).T
            bad = ~(np.abs(got - want) <= 1e-5 * scale + 1e-6)
            assert not bad.any(), f"n={n}: {bad.sum()} values off, worst {np.abs(got - want).max()}"
    finally:
        W.release()


@pytest.mark.parametrize("math", [G.MATH_PACKED, G.MATH_F32])
@pytest.mark.parametrize("qtype", [G.Q4_K, G.Q5_K, G.Q6_K, G.Q3_K, G.Q2_K, G.Q8_0, G.Q4_0, G.F16, G.F32])
def test_dense_every_type(dev, qtype, math):
    e, _ = O.block_layout(qtype)
    check(dev, qtype, 67, 1024 if e == 256 else 256, (1, 3, 8, 70), math)


@pytest.mark.parametrize("qtype", [G.Q4_K, G.Q5_K, G.Q6_K, G.Q3_K, G.Q2_K, G.Q8_0, G.Q4_0])
def test_dense_quantised_in_staging(dev, qtype):
    # 4096 columns: the call splits K into 8 slices, so under packed math each down
    # workgroup quantises its own activations (the 67-row shapes above take the
    # separate quantiser); zero blocks and partly zero blocks included
    rows, cols = 256, 4096
    e, _ = O.block_layout(qtype)
    raw = fast_random_blocks(qtype, rows * cols // e, 5 + qtype)
    W = G.DenseWeight(dev, qtype, rows, cols, raw, G.MATH_PACKED)
    try:
        deq = O.dequantize(qtype, raw, rows * cols, checked=False).reshape(rows, cols)
        for n in (1, 8, 70):
            say(f"dense {qtype} {rows}x{cols} quantised in staging, n={n}")
            xs = np.random.default_rng(n).normal(0, 1, (n, cols)).astype(np.float32)
            xs[0, :7] = 0.0
            if n > 1:
                xs[1, 32:64] = 0.0
            got = W.matmul_rows(xs)
            want = O.matmul(qtype, raw, rows, cols, xs, n, threads=8).reshape(n, rows)
            scale = np.abs(xs) @ np.abs(deq).T
            bad = ~(np.abs(got - want) <= 1e-5 * scale + 1e-6)
            assert not bad.any(), f"n={n}: {bad.sum()} values off, worst {np.abs(got - want).max()}"
    finally:
        W.release()


@pytest.mark.parametrize("qtype", [G.Q4_K, G.Q6_K, G.Q8_0, G.Q2_K])
def test_dense_prefill_on_mfma(dev, qtype):
    # rows a multiple of 512 and f32 math: the MFMA path, with a ragged last token tile
    check(dev, qtype, 1024, 2048, (64, 200), G.MATH_F32, seed=1)


def test_output_head_shape(dev):
    # a 32000-token vocabulary head over d_model 4096 in Q6_K, a decode batch of 8
    check(dev, G.Q6_K, 32000, 4096, (8,), G.MATH_PACKED, seed=2)


def test_attention_projection_shapes(dev):
    # C5's q/o (4096 x 4096) and k/v (1024 x 4096) in Q4_K
    check(dev, G.Q4_K, 4096, 4096, (1, 8), G.MATH_PACKED, seed=3)
    check(dev, G.Q4_K, 1024, 4096, (8, 512), G.MATH_F32, seed=4)


def _hip():
    """The HIP runtime the library itself links (torch bundles a runtime of its own, which
    does not share devices with this one in a process where the library came first)."""
    import ctypes as C
    h = C.CDLL("/opt/rocm/lib/libamdhip64.so.7")
    h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    h.hipFree.argtypes = [C.c_void_p]
    h.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
    h.hipStreamSynchronize.argtypes = [C.c_void_p]
    h.hipStreamDestroy.argtypes = [C.c_void_p]
    return h


def test_async_matches_sync(dev):
    import ctypes as C
    hip = _hip()
    rows, cols, n = 512, 2048, 96
    raw = fast_random_blocks(G.Q4_K, rows * cols // 256, 77)
    xs = np.random.default_rng(8).normal(0, 1, (n, cols)).astype(np.float32)
    dx, dout, st = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert hip.hipMalloc(C.byref(dx), xs.nbytes) == 0 and hip.hipMalloc(C.byref(dout), n * rows * 4) == 0
    assert hip.hipStreamCreate(C.byref(st)) == 0
    try:
        assert hip.hipMemcpy(dx, xs.ctypes.data, xs.nbytes, 1) == 0
        for math in (G.MATH_PACKED, G.MATH_F32):
            W = G.DenseWeight(dev, G.Q4_K, rows, cols, raw, math)
            try:
                want = W.matmul_rows(xs)
                W.forward_async(dx.value, n, dout.value, st.value)
                assert hip.hipStreamSynchronize(st) == 0
                got = np.empty((n, rows), np.float32)
                assert hip.hipMemcpy(got.ctypes.data, dout, got.nbytes, 2) == 0
                assert np.array_equal(bits(got), bits(want)), f"math={math}"
            finally:
                W.release()
    finally:
        hip.hipStreamDestroy(st)
        hip.hipFree(dx)
        hip.hipFree(dout)


def test_slices_add_up_to_the_forward(dev):
    # gmoe_dense_forward_slices_async: its K slices, added in slice order, are the async
    # forward's output bit for bit (packed decode with the token split, packed with
    # fewer tokens, and f32 math at a prefill size on MFMA)
    import ctypes as C
    hip = _hip()
    rows, cols = 1024, 4096
    raw = fast_random_blocks(G.Q4_K, rows * cols // 256, 78)
    nmax = 96
    dx, dout, dp = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert hip.hipMalloc(C.byref(dx), nmax * cols * 4) == 0 and hip.hipMalloc(C.byref(dout), nmax * rows * 4) == 0
    assert hip.hipMalloc(C.byref(dp), G.DenseWeight.MAX_SLICES * nmax * rows * 4) == 0
    try:
        for math, n in ((G.MATH_PACKED, 8), (G.MATH_PACKED, 3), (G.MATH_F32, 96)):
            say(f"dense slices math={math} n={n}")
            xs = np.random.default_rng(9 + n).normal(0, 1, (n, cols)).astype(np.float32)
            assert hip.hipMemcpy(dx, xs.ctypes.data, xs.nbytes, 1) == 0
            W = G.DenseWeight(dev, G.Q4_K, rows, cols, raw, math)
            try:
                W.forward_async(dx.value, n, dout.value)
                want = np.empty((n, rows), np.float32)
                assert hip.hipDeviceSynchronize() == 0
                assert hip.hipMemcpy(want.ctypes.data, dout, want.nbytes, 2) == 0
                nsl = W.forward_slices_async(dx.value, n, dp.value)
                assert 1 <= nsl <= G.DenseWeight.MAX_SLICES
                parts = np.empty((nsl, n, rows), np.float32)
                assert hip.hipDeviceSynchronize() == 0
                assert hip.hipMemcpy(parts.ctypes.data, dp, parts.nbytes, 2) == 0
                got = parts[0].copy()
                for s in range(1, nsl):
                    got = got + parts[s]
                assert np.array_equal(bits(got), bits(want)), f"math={math} n={n} nsl={nsl}"
            finally:
                W.release()
    finally:
        hip.hipFree(dx)
        hip.hipFree(dout)
        hip.hipFree(dp)


def test_from_gguf(dev, tmp_path):
    rows, cols = 256, 512
    raw = G.quantize(G.Q6_K, np.random.default_rng(1).normal(0, 0.02, rows * cols).astype(np.float32))
    path = tmp_path / "d.gguf"
    gg.write_gguf_file(path, [("general.architecture", gg.STRING, "llama")],
                       [("blk.0.attn_q.weight", [cols, rows], G.Q6_K, raw)])
    xs = np.random.default_rng(2).normal(0, 1, (4, cols)).astype(np.float32)
    with G.Gguf.open(path) as g:
        W = G.DenseWeight.from_gguf(dev, g, "blk.0.attn_q.weight")
        V = G.DenseWeight(dev, G.Q6_K, rows, cols, raw)
        try:
            assert (W.rows, W.cols) == (rows, cols)
            assert np.array_equal(bits(W.matmul_rows(xs)), bits(V.matmul_rows(xs)))
        finally:
            W.release()
            V.release()


def test_dense_refusals(dev):
    raw = np.zeros(G.byte_size(G.Q4_K, 64 * 256), np.uint8)
    with pytest.raises(G.ModelError):
        G.DenseWeight(dev, G.Q4_K, 64, 256, raw[:-1])
    with pytest.raises(G.ModelError):
        G.DenseWeight(dev, 3, 64, 256, raw)  # Q4_1: no block layout here
    W = G.DenseWeight(dev, G.Q4_K, 64, 256, raw)
    with pytest.raises(G.InferenceError):
        W.matmul_rows(np.zeros((2, 128), np.float32))
    W.release()
    with pytest.raises(G.InferenceError):
        W.matmul_rows(np.zeros((2, 256), np.float32))
