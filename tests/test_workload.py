"""The synthetic prefill workload: routing skewed to Zipf(1.1)
expert loads through one shared activation direction. CPU only: the logits here are
f64 numpy products, close enough to show the realised shares."""
import numpy as np

from garuda_amd import moe as M

ZIPF = np.array([r ** -1.1 for r in range(1, 9)])
ZIPF = ZIPF / ZIPF.sum()


def test_skew_gives_zipf_shares():
    d, ne, k, n = 1024, 8, 2, 4096
    rng = np.random.default_rng(3)
    u = M.skew_direction(11, d)
    router = M.skew_router(rng.normal(0, 0.02, ne * d).astype(np.float32), ne, d, u)
    hs = M.skew_tokens(rng.normal(0, 1, (n, d)).astype(np.float32), u)
    logits = hs.astype(np.float64) @ router.reshape(ne, d).astype(np.float64).T
    top = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    shares = np.bincount(top.ravel(), minlength=ne) / (n * k)
    assert np.abs(shares - ZIPF).max() < 0.02, shares


def test_skewed_tokens_stay_unit_normal():
    d, n = 4096, 256
    u = M.skew_direction(5, d)
    hs = M.skew_tokens(np.random.default_rng(1).normal(0, 1, (n, d)).astype(np.float32), u)
    assert np.allclose(hs.astype(np.float64) @ u, 4.0, atol=1e-3)  # the shared component
    assert abs(hs.std() - 1.0) < 0.01 and abs(hs.mean()) < 0.01
