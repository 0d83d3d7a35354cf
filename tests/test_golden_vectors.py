"""The oracle against its own committed outputs (tests/golden/oracle_vectors.npz, written by
tests/golden/make_fixtures.py): the reference tests' inputs (random_block over splitmix64 with
the seeds 0xBEEF + qtype, quant/mod.rs:1134-1160, :1184-1232) are regenerated and must equal
the stored ones, and the oracle's packed matvec and dequantisation of them must equal the
stored outputs bit for bit. A change to the oracle, or to the input generator, that moves any
value fails here."""
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import SplitMix, random_block, ref_x

GOLDEN = Path(__file__).resolve().parent / "golden" / "oracle_vectors.npz"


@pytest.fixture(scope="module")
def stored():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("qtype", O.INT8_TYPES)
def test_oracle_outputs_have_not_drifted(stored, qtype):
    elems, _ = O.block_layout(qtype)
    rows, bpr = 5, 3
    cols = bpr * elems
    rng = SplitMix(0xBEEF + qtype)
    w = np.frombuffer(b"".join(random_block(qtype, rng) for _ in range(rows * bpr)), np.uint8).copy()
    x = ref_x(rng, cols, 5)
    assert np.array_equal(w, stored[f"w_{qtype}"]), "the reference tests' weight blocks changed"
    assert np.array_equal(x.view(np.uint32), stored[f"x_{qtype}"].view(np.uint32)), "the activations changed"
    got = O.matvec(qtype, w, rows, cols, x)
    assert np.array_equal(got.view(np.uint32), stored[f"packed_{qtype}"].view(np.uint32)), "packed matvec moved"
    deq = O.dequantize(qtype, w, rows * cols)
    assert np.array_equal(deq.view(np.uint32), stored[f"deq_{qtype}"].view(np.uint32)), "dequantisation moved"


def test_every_stored_type_is_checked(stored):
    types = sorted({int(k.split("_")[1]) for k in stored})
    assert types == sorted(O.INT8_TYPES)
