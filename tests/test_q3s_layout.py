"""The Q3_K slab regrouping against the oracle, on the CPU.

The slab keeps a Q3_K unit's values regrouped (q3s_byte, q3s_word and q3s_pair in
garuda_amd/csrc/gmoe_internal.h): `k_tile_rows` writes them on the device and every Q3_K
kernel decodes them. `tests/q3s_layout_check.cpp`, built here for the host from the same
header, regroups random packed blocks and decodes every sub-block back. The quants must
be the ones the oracle's dequantisation (quant/mod.rs:840-875, pinned by the reference's
known-answer tests) multiplies: with d = 1 the oracle's value l of sub-block s is
(sc_s - 32) * q, so q = value / (sc_s - 32) exactly wherever sc_s != 32.
"""
import ctypes as C
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

ROOT = Path(__file__).resolve().parents[1]
CLANG = Path("/opt/rocm/llvm/bin/clang++")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    cxx = str(CLANG) if CLANG.exists() else shutil.which("clang++")
    if cxx is None:
        pytest.skip("no clang++ to build the host checker")
    exe = tmp_path_factory.mktemp("q3s") / "q3s_check"
    subprocess.run([cxx, "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    f"-I{ROOT / 'garuda_amd' / 'csrc'}", str(ROOT / "tests" / "q3s_layout_check.cpp"),
                    "-o", str(exe)], check=True)
    return exe


def _scales(block):
    out = (C.c_int8 * 16)()
    raw = (C.c_uint8 * 12).from_buffer_copy(bytes(block[96:108]))
    O.lib().or_unpack_q3_k_scales(raw, out)
    return np.array(out[:], dtype=np.int32)


def test_regrouped_values_are_the_blocks_quants(checker):
    rng = np.random.default_rng(2025)
    nblk = 512
    blocks = rng.integers(0, 256, (nblk, 110), dtype=np.uint8)
    blocks[:, 108:110] = np.frombuffer(np.float16(1.0).tobytes(), dtype=np.uint8)  # d = 1
    blocks[0, :96] = 0          # every q2 0 and every high bit clear: all quants -4
    blocks[1, :96] = 0xff       # every q2 3 and every high bit set: all quants 3
    got = np.frombuffer(subprocess.run([str(checker)], input=blocks.tobytes(), capture_output=True,
                                       check=True).stdout, dtype=np.int8).reshape(nblk, 256)
    assert (got[0] == -4).all() and (got[1] == 3).all()
    vals = O.dequantize(O.Q3_K, blocks.reshape(-1), nblk * 256).reshape(nblk, 16, 16)
    checked = 0
    for b in range(nblk):
        dl = _scales(blocks[b]) - 32
        for s in range(16):
            if dl[s] == 0:
                continue
            q = vals[b, s] / np.float32(dl[s])
            assert (q == np.round(q)).all()
            assert (got[b, 16 * s:16 * s + 16] == q.astype(np.int32)).all(), (b, s)
            checked += 1
    assert checked > 15 * nblk
