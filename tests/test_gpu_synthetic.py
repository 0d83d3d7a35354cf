"""garuda's synthetic engine on the GPU (MoeEngine, moe/mod.rs:67-187) against the oracle.

The layer: experts from the L2 tier (ExpertTier: expert_{id}.bin files, the missing ones
synthesised and written), the Router's gatings, rank-order combine, f32 products; routing
bit-exact and outputs within rtol 1e-3 / atol 1e-4 of oracle.feed_forward_batch over
experts made by the oracle's own synthesize_expert. The experts 0, 3, 6 and 7 are written
first, byte for byte the reference's models/l2_cache files (their SHA-256 pins the oracle's
generator, tests/test_oracle_path.py), so those come from files.

The engine: BASELINE configuration 1's shape (garuda_amd.synthetic.SyntheticEngine)
decoding against oracle.model.ModelOracle built from the oracle's generators, f32 math:
every step's logits within 1e-3 of their size and the same greedy token wherever the
top two logits are apart."""
from __future__ import annotations

import numpy as np
import pytest

import garuda_amd as G
from garuda_amd.synthetic import SyntheticEngine
from garuda_amd.tiers import SEED_ROUTER, ExpertTier
from oracle import oracle as O
from oracle.model import engine_experts as oracle_experts, synthetic_engine
from tests.test_gpu_parity import ATOL, RTOL, bits, say

pytestmark = pytest.mark.gpu

D, F, NE, K = 128, 256, 8, 2  # ModelDims::default (core/mod.rs:68-82)


@pytest.fixture(scope="module")
def dev():
    d = G.Device(0, slab_bytes=256 << 20)
    yield d
    d.close()


def write_reference_fixtures(directory):
    for e in (0, 3, 6, 7):  # byte for byte models/l2_cache/expert_{0,3,6,7}.bin
        g, u, dn = O.synthesize_expert(e)
        (directory / f"expert_{e}.bin").write_bytes(np.concatenate([g, u, dn]).astype("<f4").tobytes())


@pytest.mark.parametrize("gating", [G.GATING_MIXTRAL, G.GATING_DEEPSEEK, G.GATING_QWEN])
def test_engine_layer_from_the_l2_tier(dev, tmp_path, gating):
    write_reference_fixtures(tmp_path)
    router = O.seeded(SEED_ROUTER, NE * D, O.lib().or_bound(D))
    gate, up, down = oracle_experts(D, F, range(NE))
    L = dict(d=D, f=F, ne=NE, k=K, gating=gating, combine=1, packed=0, router=router,
             qtypes=(O.F32,) * 3, gate=gate, up=up, down=down)
    rng = np.random.default_rng(gating)
    with ExpertTier(tmp_path, D, F, NE) as tier:
        c = tier.counts()
        assert (c.l2, c.synthesised) == (4, NE - 4)
        layer = tier.layer(dev, router, K, gating, G.COMBINE_RANK_ORDER)
        try:
            for n in (1, 2, 7, 33):
                say(f"engine layer gating={gating} n={n}")
                hs = rng.normal(0, 1, (n, D)).astype(np.float32)
                hs[0] = hs[0] / np.sqrt(np.mean(hs[0] ** 2))  # a normed row, as moe_ffn sees it
                out, ids, w = layer.feed_forward_batch(hs)
                wout, wids, ww = O.feed_forward_batch(L, hs)
                assert np.array_equal(ids, wids) and np.array_equal(bits(w), bits(ww))
                assert np.allclose(out, wout, rtol=RTOL, atol=ATOL), np.abs(out - wout).max()
        finally:
            layer.release()


def test_engine_layer_restages_evicted_experts_from_the_tier(tmp_path):
    write_reference_fixtures(tmp_path)
    router = O.seeded(SEED_ROUTER, NE * D, O.lib().or_bound(D))
    gate, up, down = oracle_experts(D, F, range(NE))
    L = dict(d=D, f=F, ne=NE, k=K, gating=1, combine=1, packed=0, router=router, qtypes=(O.F32,) * 3,
             gate=gate, up=up, down=down)
    per = 3 * F * D * 4
    rng = np.random.default_rng(5)
    # room for four experts: the most one call of two tokens at top-2 routes to
    with G.Device(0, slab_bytes=4 * per + (1 << 16)) as small, ExpertTier(tmp_path, D, F, NE) as tier:
        layer = tier.layer(small, router, K)
        try:
            for step in range(6):
                hs = rng.normal(0, 1, (2, D)).astype(np.float32)
                out, ids, _ = layer.feed_forward_batch(hs)
                wout, wids, _ = O.feed_forward_batch(L, hs)
                assert np.array_equal(ids, wids) and np.allclose(out, wout, rtol=RTOL, atol=ATOL)
            assert small.slab_stats().evictions > 0
        finally:
            layer.release()


def test_c1_engine_decodes_as_the_oracle(dev, tmp_path):
    # 4 layers, d 256, 8 query / 2 kv heads of 32, 8 experts
    # top-2 of 512, vocab 512; two sequences, 6 prompt tokens then greedy decoding
    dims = dict(n_layers=4, d=256, nh=8, nkv=2, hd=32, f=512, ne=8, k=2, vocab=512)
    orc = synthetic_engine(**dims, max_positions=256)
    with SyntheticEngine(dev, tmp_path, n_layers=4, d_model=256, n_heads=8, n_kv_heads=2, head_dim=32, d_ff=512,
                         n_experts=8, top_k=2, vocab=512, max_positions=256) as eng:
        seqs = [eng.open_seq(), eng.open_seq()]
        prompt = np.random.default_rng(1).integers(0, 512, (2, 6)).astype(np.uint32)
        toks = prompt[:, 0]
        ambiguous = set()
        for step in range(14):
            say(f"c1 engine step {step}")
            gn, gl = eng.step(seqs, toks, want_logits=True)
            on, ol = orc.decode_step(seqs, toks)
            ambiguous |= {i for i, m in enumerate(orc.last_margins) if m < 1e-4}
            for i in range(2):
                if i in ambiguous:
                    continue
                scale = float(np.abs(ol[i]).max())
                err = float(np.abs(gl[i] - ol[i]).max())
                assert err <= 1e-3 * scale, (step, i, err, scale)
                top2 = np.sort(ol[i])[-2:]
                if top2[1] - top2[0] > 4e-3 * scale:
                    assert gn[i] == on[i], (step, i)
            nxt = prompt[:, step + 1] if step + 1 < prompt.shape[1] else on
            toks = np.asarray(nxt, np.uint32)
        assert len(ambiguous) < 2


def test_engine_layer_over_lazy_l2_l3_tiers(tmp_path):
    """MemoryManager's full path under the slab (memory/mod.rs:114-146): a layer whose
    experts are fetched when routed. Experts 0, 3, 6 and 7 sit in L3 only, the others
    nowhere: a routed L3 expert is promoted into L2, a routed absent one synthesised into
    L2, an unrouted one never loaded; after an eviction the expert comes back from L2.
    Outputs and routing as the oracle's, bit-exact routing."""
    l2, l3 = tmp_path / "l2", tmp_path / "l3"
    l2.mkdir()
    l3.mkdir()
    write_reference_fixtures(l3)
    router = O.seeded(SEED_ROUTER, NE * D, O.lib().or_bound(D))
    gate, up, down = oracle_experts(D, F, range(NE))
    L = dict(d=D, f=F, ne=NE, k=K, gating=G.GATING_MIXTRAL, combine=1, packed=0, router=router,
             qtypes=(O.F32,) * 3, gate=gate, up=up, down=down)
    per = 3 * F * D * 4
    rng = np.random.default_rng(11)
    # room for two experts: a one-token call at top-2, so every call evicts
    with G.Device(0, slab_bytes=2 * per + (1 << 16)) as small, ExpertTier(l2, D, F, NE, l3=l3) as tier:
        layer = tier.layer(small, router, K, G.GATING_MIXTRAL, G.COMBINE_RANK_ORDER)
        try:
            assert not any(layer.is_resident(e) for e in range(NE))  # nothing loaded at registration
            assert tier.counts().l2 + tier.counts().l3 + tier.counts().synthesised == 0
            seen = []
            for step in range(10):
                say(f"lazy tiers step {step}")
                hs = rng.normal(0, 1, (1, D)).astype(np.float32)
                before = {e: tier.locate(e) for e in range(NE)}
                c0 = tier.counts()
                resident = [e for e in range(NE) if layer.is_resident(e)]
                out, ids, w = layer.feed_forward_batch(hs)
                wout, wids, ww = O.feed_forward_batch(L, hs)
                assert np.array_equal(ids, wids) and np.array_equal(bits(w), bits(ww))
                assert np.allclose(out, wout, rtol=RTOL, atol=ATOL), np.abs(out - wout).max()
                c1 = tier.counts()
                loaded = [int(e) for e in ids.reshape(-1) if int(e) not in resident]
                want = {G.TIER_L2: 0, G.TIER_L3: 0, G.TIER_SYNTHESISED: 0}
                for e in loaded:
                    want[before[e]] += 1
                assert (c1.l2 - c0.l2, c1.l3 - c0.l3, c1.synthesised - c0.synthesised) == \
                    (want[G.TIER_L2], want[G.TIER_L3], want[G.TIER_SYNTHESISED]), (step, loaded, before)
                for e in loaded:
                    assert tier.locate(e) == G.TIER_L2  # promoted or materialised into L2
                seen += [int(e) for e in ids.reshape(-1)]
            for e in set(range(NE)) - set(seen):
                assert not (l2 / f"expert_{e}.bin").exists()  # never routed, never loaded
            assert small.slab_stats().evictions > 0 and tier.counts().l2 > 0
        finally:
            layer.release()
