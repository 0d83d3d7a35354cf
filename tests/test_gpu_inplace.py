"""A layer call whose output overwrites its input (out == hs) through the C-ABI.

At decode batches with top-k <= 2 the front end zeroes the output rows while it reads the
activations, and the down product adds into them; an output that aliases the input takes
the launch sequence with the separate combine instead, which writes the output last. The
result must be the reference's (llama/mod.rs:903-1020) all the same: routing bit-exact,
outputs within rtol 1e-3 / atol 1e-4. Device buffers come from the HIP runtime the
library links."""
import ctypes as C
import os

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import _lib
from oracle import oracle as O
from tests.test_gpu_dense import _hip
from tests.test_gpu_parity import ATOL, RTOL, bits, make_layer, oracle_layer, say

pytestmark = pytest.mark.gpu


def test_output_overwriting_the_input():
    d, f, ne, k = 512, 1024, 8, 2
    rng = np.random.default_rng(91)
    router, mats = make_layer(rng, d, f, ne, G.Q4_K, G.Q4_K)
    lib, hip = _lib.lib(), _hip()
    hip.hipDeviceSynchronize.argtypes = []
    L = oracle_layer(d, f, ne, k, router, mats, (G.Q4_K,) * 3, G.MATH_PACKED)
    with G.Device(0, slab_bytes=1 << 30) as dev:
        layer = G.MoeLayer(dev, d, f, ne, k, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
        bufs = []
        try:
            for n in (1, 8):
                say(f"in-place layer call, n={n}")
                hs = rng.normal(0, 1, (n, d)).astype(np.float32)
                p, ids, w = C.c_void_p(), C.c_void_p(), C.c_void_p()
                for q, nbytes in ((p, hs.nbytes), (ids, n * k * 4), (w, n * k * 4)):
                    assert hip.hipMalloc(C.byref(q), nbytes) == 0
                    bufs.append(q)
                assert hip.hipMemcpy(p, hs.ctypes.data, hs.nbytes, 1) == 0
                assert hip.hipDeviceSynchronize() == 0
                rc = lib.gmoe_ffn_forward_async(dev.handle, layer.id, p, None, n, p, ids, w, None)
                assert rc == 0, lib.gmoe_last_error()
                assert hip.hipDeviceSynchronize() == 0
                out = np.empty((n, d), np.float32)
                gid, gw = np.empty((n, k), np.uint32), np.empty((n, k), np.float32)
                for arr, q in ((out, p), (gid, ids), (gw, w)):
                    assert hip.hipMemcpy(arr.ctypes.data, q, arr.nbytes, 2) == 0
                wout, wids, ww = O.feed_forward_batch(L, hs, threads=min(16, len(os.sched_getaffinity(0))))
                assert np.array_equal(gid, wids) and np.array_equal(bits(gw), bits(ww))
                assert np.allclose(out, wout, rtol=RTOL, atol=ATOL), f"n={n} max err {np.abs(out - wout).max()}"
        finally:
            assert hip.hipDeviceSynchronize() == 0
            for q in bufs:
                hip.hipFree(q)
            layer.release()
