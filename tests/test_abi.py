"""CPU checks of the native library: it loads, exports every entry point the header
declares, and its host-side helpers (quantisers, generator) are sound. No GPU calls."""
import re
from pathlib import Path

import numpy as np
import pytest

from garuda_amd import _lib
from garuda_amd import moe as M
from oracle import oracle as O

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "garuda_moe.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"typedef[^;]*\(\s*\*[^;]*;", "", text)  # function-pointer types (callbacks)
    return sorted(set(re.findall(r"\b(gmoe_[a-z_0-9]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.lib()
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) == set(_lib.SIGNATURES), "ctypes table and header disagree"
    assert lib.gmoe_abi_version() == 6
    assert lib.gmoe_last_invalid_token() == 0xFFFFFFFF  # none yet on this thread


def test_library_leaves_no_internal_symbol_undefined():
    """A shared library links with undefined symbols; one of the library's own (namespace
    gmoe) would only fail when the library is loaded on the GPU box."""
    import shutil
    import subprocess
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm is not installed")
    out = subprocess.run([nm, "-D", "--undefined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    own = [l.split()[-1] for l in out.splitlines() if l.split() and l.split()[-1].startswith("_ZN4gmoe")]
    assert not own, own


@pytest.mark.parametrize("qtype", [M.Q4_K, M.Q5_K, M.Q6_K, M.Q3_K, M.Q2_K, M.Q8_0, M.Q4_0, M.F16, M.F32])
def test_quantiser_round_trips_through_the_reference_decoder(qtype):
    x = M.fill_gaussian(1234 + qtype, 256 * 64, 0.0, 0.02)
    raw = M.quantize(qtype, x)
    assert raw.size == O.byte_size(qtype, x.size)
    y = O.dequantize(qtype, raw, x.size)
    # error per element within two steps of its 256-block's scale, a step being
    # (max |x| over the block) / levels and levels the format's positive quant range;
    # one step for rounding, one for the sub-scale rounding and the clamp at the top code
    levels = {M.Q4_K: 15, M.Q5_K: 31, M.Q6_K: 31, M.Q3_K: 3, M.Q2_K: 3, M.Q8_0: 127, M.Q4_0: 7,
              M.F16: 2 ** 10, M.F32: 2 ** 23}[qtype]
    blk = np.abs(x).reshape(-1, 256).max(axis=1).repeat(256)
    assert (np.abs(y - x) <= 2 * blk / levels + 1e-7).all()
    rel = np.linalg.norm(y - x) / np.linalg.norm(x)
    assert rel < {M.Q2_K: 0.5, M.Q3_K: 0.3}.get(qtype, 0.1)


def test_gaussian_generator_is_deterministic_and_standard():
    a = M.fill_gaussian(7, 1 << 20)
    b = M.fill_gaussian(7, 1 << 20, threads=1)
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    assert not np.array_equal(a, M.fill_gaussian(8, 1 << 20))


def test_byte_size_and_refusals():
    assert M.byte_size(M.Q4_K, 4096) == 2304
    assert M.byte_size(M.Q6_K, 2048) == 1680
    assert M.byte_size(M.Q8_0, 768) == 816
    with pytest.raises(M.ModelError):
        M.byte_size(M.Q4_K, 100)
    with pytest.raises(M.ModelError):
        M.byte_size(3, 32)
