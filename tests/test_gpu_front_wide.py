"""The front end for 64 < ne <= 256 experts (k_front_wide) through the C-ABI.

One wave per token gates it with every ordered sum in expert order (router/mod.rs:58-118,
llama/mod.rs:939-949) and quantises its activations; the last workgroup dispatches all
pairs as a stable counting sort (llama/mod.rs:966-972) with per-wave ranks. Routing ids
and weights must be bit-exact, outputs within rtol 1e-3 / atol 1e-4.
"""
import numpy as np
import pytest

import garuda_amd as G
from tests.test_gpu_parity import check_layer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=2 << 30)
    yield d
    d.close()


@pytest.mark.parametrize("gating,combine", [(0, 0), (1, 1), (2, 1), (3, 0)])
def test_wide_front_sequential_logits(dev, gating, combine):
    # no logits given: the reference's sequential router dots, then each gating rule
    check_layer(dev, 256, 256, 128, 8, (G.Q4_K,) * 3, (1, 5, 64), G.MATH_PACKED, gating=gating, combine=combine,
                seed=90 + gating)


def test_wide_front_ragged_expert_count_with_ties(dev):
    # 200 experts (lanes hold 4 experts, the last partly empty), logits with ties
    check_layer(dev, 256, 256, 200, 6, (G.Q6_K, G.Q6_K, G.Q8_0), (3, 70), G.MATH_PACKED, seed=95, tie_logits=True)


def test_wide_front_given_logits_c4_like(dev):
    # C4's routing: 128 experts, top-8, uniform logits scaled by 4
    check_layer(dev, 512, 256, 128, 8, (G.Q6_K, G.Q6_K, G.Q8_0), (1, 8, 64), G.MATH_PACKED, seed=96, logits_scale=4.0)


def test_wide_front_prefill_tiles(dev):
    # f32 math at 300 tokens: the dispatch also writes the MFMA prefill's token tiles
    check_layer(dev, 512, 512, 128, 4, (G.Q4_K,) * 3, (300,), G.MATH_F32, seed=97, logits_scale=4.0)


def test_wide_front_many_dispatch_rounds(dev):
    # 600 tokens of top-8 over 96 experts: 4800 pairs, ten rounds of the dispatch
    check_layer(dev, 256, 256, 96, 8, (G.Q4_K,) * 3, (600,), G.MATH_PACKED, seed=98, sample=40)
