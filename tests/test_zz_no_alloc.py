"""The allocation-free forward (gmoe_ffn_forward_noalloc) through the C-ABI against the
arena-backed gmoe_ffn_forward_async on the same inputs: two calls in a row, the second
smaller, each bit-identical in outputs, routed ids and weights (both run the same
kernels), plus a call too large for the static scratch, refused before any device work.
Device buffers come from the HIP runtime the library links."""
import ctypes as C

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import _lib
from tests.test_gpu_dense import _hip
from tests.test_gpu_parity import make_layer, say

pytestmark = pytest.mark.gpu


def test_noalloc_forward_matches_the_async_forward():
    d, f, ne, k = 512, 8192, 8, 2  # f 8192: the down product runs in several K slices
    rng = np.random.default_rng(77)
    router, mats = make_layer(rng, d, f, ne, G.Q4_K, G.Q4_K)
    lib, hip = _lib.lib(), _hip()
    hip.hipDeviceSynchronize.argtypes = []
    bufs = []

    def dalloc(nbytes, fill=None):
        p = C.c_void_p()
        assert hip.hipMalloc(C.byref(p), nbytes) == 0
        bufs.append(p)
        if fill is not None:
            assert hip.hipMemcpy(p, np.ascontiguousarray(fill).ctypes.data, nbytes, 1) == 0
        return p

    def fetch(p, shape, dtype):
        a = np.empty(shape, dtype)
        assert hip.hipDeviceSynchronize() == 0
        assert hip.hipMemcpy(a.ctypes.data, p, a.nbytes, 2) == 0
        return a

    with G.Device(0, slab_bytes=1 << 30) as dev:
        layer = G.MoeLayer(dev, d, f, ne, k, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
        try:
            for n in (8, 3):
                say(f"no-alloc forward, n={n}")
                hs = dalloc(n * d * 4, rng.normal(0, 1, (n, d)).astype(np.float32))
                got = []
                for fn in (lib.gmoe_ffn_forward_async, lib.gmoe_ffn_forward_noalloc):
                    out = dalloc(n * d * 4, np.full((n, d), np.nan, np.float32))
                    ids = dalloc(n * k * 4, np.full((n, k), 0xFFFFFFFF, np.uint32))
                    w = dalloc(n * k * 4, np.full((n, k), np.nan, np.float32))
                    assert hip.hipDeviceSynchronize() == 0
                    rc = fn(dev.handle, layer.id, hs, None, n, out, ids, w, None)
                    assert rc == 0, lib.gmoe_last_error()
                    got.append((fetch(out, (n, d), np.float32), fetch(ids, (n, k), np.uint32),
                                fetch(w, (n, k), np.float32)))
                (oa, ia, wa), (ob, ib, wb) = got
                assert np.isfinite(ob).all() and (ib < ne).all()
                assert np.array_equal(ia, ib)
                assert np.array_equal(wa.view(np.uint32), wb.view(np.uint32))
                assert np.array_equal(oa.view(np.uint32), ob.view(np.uint32))
            # a call whose launch sequence needs more than the static scratch is refused
            big = 4096
            hs = dalloc(big * d * 4)
            out = dalloc(big * d * 4)
            rc = lib.gmoe_ffn_forward_noalloc(dev.handle, layer.id, hs, None, big, out, None, None, None)
            assert rc == 2 and b"allocation-free" in lib.gmoe_last_error()
        finally:
            assert hip.hipDeviceSynchronize() == 0
            for p in bufs:
                hip.hipFree(p)
            layer.release()
