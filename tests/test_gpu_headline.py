"""GPU parity at the BASELINE configurations' own shapes, through the C-ABI.

The decode path behind the C2 and C5 bench numbers splits each down-product row over K
slices once d_ff is wide (down_ksg: 2 slices at f 4096, 4 at 8192, up to 7 at 14336
for Q4_K) and adds the slices in the combine. These tests run that path at its real
widths against the oracle's restatement of feed_forward_batch (llama/mod.rs:903-1020):
routing ids and weights bit-exact, outputs within rtol 1e-3 / atol 1e-4.
"""
import numpy as np
import pytest

import garuda_amd as G
from garuda_amd import moe as M
from tests.test_gpu_parity import check_layer, make_layer, say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=3 << 30)
    yield d
    d.close()


@pytest.mark.parametrize("f", [4096, 8192, 14336])
def test_down_product_split_over_k_slices(dev, f):
    # d 256 keeps the oracle cheap; f sets the down rows' width: 2, 4 and 7 K slices at
    # up to 4 (token, expert) pairs, and as many at 8 and 20 tokens
    check_layer(dev, 256, f, 8, 2, (G.Q4_K,) * 3, (1, 2, 4, 8, 20), G.MATH_PACKED, seed=40 + f // 1024)


def test_down_product_split_other_types(dev):
    check_layer(dev, 256, 14336, 8, 2, (G.Q3_K, G.Q3_K, G.Q4_K), (1, 8), G.MATH_PACKED, seed=41)
    check_layer(dev, 256, 8192, 8, 2, (G.Q6_K, G.Q6_K, G.Q8_0), (2, 8), G.MATH_PACKED, seed=42)


def test_c2_layer_decode_batches(dev):
    # d 4096, f 14336, 8 experts, top-2, Q4_K, packed math, batch 1-8
    check_layer(dev, 4096, 14336, 8, 2, (G.Q4_K,) * 3, (1, 2, 4, 8), G.MATH_PACKED, seed=43)


def test_c2_layer_decode_f32_math(dev):
    check_layer(dev, 4096, 14336, 8, 2, (G.Q4_K,) * 3, (1, 8), G.MATH_F32, seed=44)


def test_c5_layer_slice(dev):
    # BASELINE config 5's MoE layer: Q3_K gate/up, Q4_K down, 8 concurrent decode tokens
    check_layer(dev, 4096, 14336, 8, 2, (G.Q3_K, G.Q3_K, G.Q4_K), (1, 8), G.MATH_PACKED, seed=45)


def test_c3_shape_packed_prefill_sampled(dev):
    # BASELINE config 3 under packed math (mmap = true): 512 Zipf-skewed tokens through the
    # whole layer on the GPU, 24 of them compared with the oracle
    check_layer(dev, 4096, 14336, 8, 2, (G.Q4_K,) * 3, (512,), G.MATH_PACKED, seed=46, zipf=True, sample=24)


def test_c4_routing_beyond_one_launch(dev):
    # 128 experts, top-8, logits given: 6000 tokens make 48000 (token, expert) pairs, which
    # run as two launch sequences; 40 tokens spread over both are compared
    check_layer(dev, 256, 256, 128, 8, (G.Q6_K, G.Q6_K, G.Q8_0), (6000,), G.MATH_PACKED, logits_scale=4.0,
                seed=47, sample=40)


def test_lru_evicts_the_least_recently_routed_expert():
    """ExpertCache::get marks only the expert it returns (cache/mod.rs:70-84): a call
    touches its routed experts in token, then rank order, and the others keep their
    place. Layer A fills the slab; layer B's first call must evict A's two least recently
    routed experts."""
    d, f, ne, k = 256, 512, 8, 2
    rng = np.random.default_rng(48)
    ra, ma = make_layer(rng, d, f, ne, G.Q4_K, G.Q4_K)
    rb, mb = make_layer(rng, d, f, ne, G.Q4_K, G.Q4_K)
    per = sum(M.byte_size(G.Q4_K, f * d) for _ in range(3))
    with G.Device(0, slab_bytes=ne * per + (1 << 16)) as small:
        A = G.MoeLayer(small, d, f, ne, k, ra, ma["gate"], ma["up"], ma["down"], (G.Q4_K,) * 3)
        B = G.MoeLayer(small, d, f, ne, k, rb, mb["gate"], mb["up"], mb["down"], (G.Q4_K,) * 3)
        assert all(A.is_resident(e) for e in range(ne)) and not any(B.is_resident(e) for e in range(ne))
        order = list(range(ne))  # A was staged expert by expert
        _, ids, _ = A.feed_forward_batch(rng.normal(0, 1, (1, d)).astype(np.float32))
        for e in ids.reshape(-1).tolist():
            order.remove(e)
            order.append(e)
        _, idb, _ = B.feed_forward_batch(rng.normal(0, 1, (1, d)).astype(np.float32))
        victims = order[:len(np.unique(idb))]
        say(f"A routed {ids.tolist()}, B routed {idb.tolist()}, expected victims {victims}")
        for e in range(ne):
            assert A.is_resident(e) == (e not in victims), e
        assert all(B.is_resident(e) for e in np.unique(idb))
        B.release()
        A.release()
