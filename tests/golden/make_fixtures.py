"""Writes the committed golden files under tests/golden/. Run from the repo root:

    python tests/golden/make_fixtures.py [--reference /root/reference]

1. l2_cache_experts.json — SHA-256 and excerpts of the reference's data fixtures
   models/l2_cache/expert_{0,3,6,7}.bin (f32 LE, gate|up|down of
   weights::synthesize_expert(id, ModelDims::default()), weights/mod.rs:98-120).
   Data only; the files are read, nothing of the reference is run.
2. oracle_vectors.npz — the oracle's outputs on the reference tests' own inputs
   (random_block / splitmix64 seeds 0xBEEF+qtype, quant/mod.rs:1184-1232), so a later
   change to the oracle that moves any of them is caught.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402
from tests.helpers import SplitMix, random_block, ref_x  # noqa: E402

OUT = Path(__file__).resolve().parent


def l2_fixture(ref: Path) -> None:
    out = {}
    for eid in (0, 3, 6, 7):
        raw = (ref / "models" / "l2_cache" / f"expert_{eid}.bin").read_bytes()
        v = np.frombuffer(raw, dtype="<f4")
        n = 128 * 256
        out[str(eid)] = {
            "bytes": len(raw),
            "sha256": hashlib.sha256(raw).hexdigest(),
            "gate_head": v[:8].tolist(),
            "up_head": v[n:n + 8].tolist(),
            "down_head": v[2 * n:2 * n + 8].tolist(),
            "down_tail": v[-8:].tolist(),
        }
    (OUT / "l2_cache_experts.json").write_text(json.dumps(out, indent=1))


def oracle_vectors() -> None:
    arrs = {}
    for qtype in O.INT8_TYPES:
        elems, _ = O.block_layout(qtype)
        rows, bpr = 5, 3
        cols = bpr * elems
        rng = SplitMix(0xBEEF + qtype)
        w = np.frombuffer(b"".join(random_block(qtype, rng) for _ in range(rows * bpr)), np.uint8).copy()
        x = ref_x(rng, cols, 5)
        arrs[f"w_{qtype}"] = w
        arrs[f"x_{qtype}"] = x
        arrs[f"packed_{qtype}"] = O.matvec(qtype, w, rows, cols, x)
        arrs[f"deq_{qtype}"] = O.dequantize(qtype, w, rows * cols)
    np.savez_compressed(OUT / "oracle_vectors.npz", **arrs)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    a = ap.parse_args()
    ref = Path(a.reference)
    if (ref / "models" / "l2_cache").exists():
        l2_fixture(ref)
    oracle_vectors()
    print("wrote", sorted(p.name for p in OUT.iterdir()))
