"""The allocation-free forward (gmoe_ffn_forward_noalloc) through the C-ABI against the
arena-backed gmoe_ffn_forward_async on the same inputs: two calls in a row, the second
smaller, each bit-identical in outputs, routed ids and weights (both run the same
kernels), plus a call too large for the static scratch, refused before any device work.
The property the entry point exists for is checked too: the device's free memory
(hipMemGetInfo) does not move across a call, calls from two contexts on two streams
without a synchronisation between them are ordered on the shared array (each still equals
the async forward), and a call captured into a HIP graph replays to the same result
several times with eager work between the replays. Device buffers come from the HIP
runtime the library links."""
import ctypes as C

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import _lib
from tests.test_gpu_dense import _hip
from tests.test_gpu_parity import make_layer, say

pytestmark = pytest.mark.gpu


def _runtime():
    hip = _hip()
    hip.hipDeviceSynchronize.argtypes = []
    hip.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    hip.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    hip.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    hip.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]
    hip.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    hip.hipGraphExecDestroy.argtypes = [C.c_void_p]
    hip.hipGraphDestroy.argtypes = [C.c_void_p]
    return hip


class Bufs:
    def __init__(self, hip):
        self.hip, self.ps = hip, []

    def alloc(self, nbytes, fill=None):
        p = C.c_void_p()
        assert self.hip.hipMalloc(C.byref(p), nbytes) == 0
        self.ps.append(p)
        if fill is not None:
            assert self.hip.hipMemcpy(p, np.ascontiguousarray(fill).ctypes.data, nbytes, 1) == 0
        return p

    def fetch(self, p, shape, dtype):
        a = np.empty(shape, dtype)
        assert self.hip.hipDeviceSynchronize() == 0
        assert self.hip.hipMemcpy(a.ctypes.data, p, a.nbytes, 2) == 0
        return a

    def free(self):
        assert self.hip.hipDeviceSynchronize() == 0
        for p in self.ps:
            self.hip.hipFree(p)


def _free_bytes(hip):
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipDeviceSynchronize() == 0
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def test_noalloc_forward_matches_the_async_forward():
    d, f, ne, k = 512, 8192, 8, 2  # f 8192: the down product runs in several K slices
    rng = np.random.default_rng(77)
    router, mats = make_layer(rng, d, f, ne, G.Q4_K, G.Q4_K)
    lib, hip = _lib.lib(), _runtime()
    B = Bufs(hip)
    with G.Device(0, slab_bytes=1 << 30) as dev:
        layer = G.MoeLayer(dev, d, f, ne, k, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
        try:
            for n in (8, 3):
                say(f"no-alloc forward, n={n}")
                hs = B.alloc(n * d * 4, rng.normal(0, 1, (n, d)).astype(np.float32))
                got = []
                for fn in (lib.gmoe_ffn_forward_async, lib.gmoe_ffn_forward_noalloc):
                    out = B.alloc(n * d * 4, np.full((n, d), np.nan, np.float32))
                    ids = B.alloc(n * k * 4, np.full((n, k), 0xFFFFFFFF, np.uint32))
                    w = B.alloc(n * k * 4, np.full((n, k), np.nan, np.float32))
                    assert hip.hipDeviceSynchronize() == 0
                    before = _free_bytes(hip)
                    rc = fn(dev.handle, layer.id, hs, None, n, out, ids, w, None)
                    assert rc == 0, lib.gmoe_last_error()
                    if fn is lib.gmoe_ffn_forward_noalloc:
                        assert _free_bytes(hip) == before, "the allocation-free call changed the free device memory"
                    got.append((B.fetch(out, (n, d), np.float32), B.fetch(ids, (n, k), np.uint32),
                                B.fetch(w, (n, k), np.float32)))
                (oa, ia, wa), (ob, ib, wb) = got
                assert np.isfinite(ob).all() and (ib < ne).all()
                assert np.array_equal(ia, ib)
                assert np.array_equal(wa.view(np.uint32), wb.view(np.uint32))
                assert np.array_equal(oa.view(np.uint32), ob.view(np.uint32))
            # a call whose launch sequence needs more than the static scratch is refused
            big = 4096
            hs = B.alloc(big * d * 4)
            out = B.alloc(big * d * 4)
            rc = lib.gmoe_ffn_forward_noalloc(dev.handle, layer.id, hs, None, big, out, None, None, None)
            assert rc == 2 and b"allocation-free" in lib.gmoe_last_error()
        finally:
            B.free()
            layer.release()


def test_noalloc_calls_from_two_contexts_on_two_streams_are_ordered():
    d, f, ne, k, n = 512, 4096, 8, 2, 6
    rng = np.random.default_rng(78)
    lib, hip = _lib.lib(), _runtime()
    B = Bufs(hip)
    with G.Device(0, slab_bytes=1 << 30) as da, G.Device(0, slab_bytes=1 << 30) as db:
        layers, refs, ins = [], [], []
        try:
            for dev in (da, db):
                router, mats = make_layer(rng, d, f, ne, G.Q4_K, G.Q4_K)
                L = G.MoeLayer(dev, d, f, ne, k, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
                layers.append(L)
                hs = B.alloc(n * d * 4, rng.normal(0, 1, (n, d)).astype(np.float32))
                out = B.alloc(n * d * 4)
                assert lib.gmoe_ffn_forward_async(dev.handle, L.id, hs, None, n, out, None, None, None) == 0
                refs.append(B.fetch(out, (n, d), np.float32))
                ins.append(hs)
            streams = [C.c_void_p(), C.c_void_p()]
            for s in streams:
                assert hip.hipStreamCreate(C.byref(s)) == 0
            outs = [[B.alloc(n * d * 4, np.full((n, d), np.nan, np.float32)) for _ in range(4)] for _ in range(2)]
            assert hip.hipDeviceSynchronize() == 0
            for r in range(4):  # alternating contexts and streams, no synchronisation between calls
                for i, dev in enumerate((da, db)):
                    rc = lib.gmoe_ffn_forward_noalloc(dev.handle, layers[i].id, ins[i], None, n, outs[i][r], None,
                                                      None, streams[i])
                    assert rc == 0, lib.gmoe_last_error()
            for i in range(2):
                for r in range(4):
                    got = B.fetch(outs[i][r], (n, d), np.float32)
                    assert np.array_equal(got.view(np.uint32), refs[i].view(np.uint32)), (i, r)
            for s in streams:
                hip.hipStreamDestroy(s)
        finally:
            B.free()
            for L in layers:
                L.release()


def test_noalloc_call_under_graph_capture_replays():
    d, f, ne, k, n = 512, 4096, 8, 2, 5
    rng = np.random.default_rng(79)
    router, mats = make_layer(rng, d, f, ne, G.Q4_K, G.Q4_K)
    lib, hip = _lib.lib(), _runtime()
    B = Bufs(hip)
    with G.Device(0, slab_bytes=1 << 30) as dev:
        layer = G.MoeLayer(dev, d, f, ne, k, router, mats["gate"], mats["up"], mats["down"], (G.Q4_K,) * 3)
        graph, exe, st = C.c_void_p(), C.c_void_p(), C.c_void_p()
        try:
            hs = B.alloc(n * d * 4, rng.normal(0, 1, (n, d)).astype(np.float32))
            ref = B.alloc(n * d * 4)
            assert lib.gmoe_ffn_forward_async(dev.handle, layer.id, hs, None, n, ref, None, None, None) == 0
            want = B.fetch(ref, (n, d), np.float32)
            out = B.alloc(n * d * 4, np.full((n, d), np.nan, np.float32))
            assert hip.hipStreamCreate(C.byref(st)) == 0
            # an eager call first (one-time set-up of the kernels), then the capture
            assert lib.gmoe_ffn_forward_noalloc(dev.handle, layer.id, hs, None, n, out, None, None, st) == 0
            assert hip.hipStreamSynchronize(st) == 0
            assert hip.hipStreamBeginCapture(st, 1) == 0  # thread-local capture mode
            rc = lib.gmoe_ffn_forward_noalloc(dev.handle, layer.id, hs, None, n, out, None, None, st)
            assert hip.hipStreamEndCapture(st, C.byref(graph)) == 0
            assert rc == 0, lib.gmoe_last_error()
            assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
            other = B.alloc(n * d * 4)
            for r in range(3):
                say(f"graph replay {r}")
                assert hip.hipMemcpy(out, np.full((n, d), np.nan, np.float32).ctypes.data, n * d * 4, 1) == 0
                assert hip.hipGraphLaunch(exe, st) == 0
                assert hip.hipStreamSynchronize(st) == 0
                got = B.fetch(out, (n, d), np.float32)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), r
                # eager work between the replays
                assert lib.gmoe_ffn_forward_async(dev.handle, layer.id, hs, None, n, other, None, None, None) == 0
                assert hip.hipDeviceSynchronize() == 0
        finally:
            if exe:
                hip.hipGraphExecDestroy(exe)
            if graph:
                hip.hipGraphDestroy(graph)
            if st:
                hip.hipStreamDestroy(st)
            B.free()
            layer.release()
