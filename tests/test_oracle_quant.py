"""Pins the oracle's quant restatement against the reference's own tests.

Each test restates one test of garuda/src/quant/mod.rs:901-1417 (cited per test) on
the oracle, with the reference's inputs, seeds and tolerances, plus checks that the
mathematics fixes where the reference has none (exhaustive f16, closed-form Q3_K).
"""
import struct

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import SplitMix, half_bits, random_block, random_rows, ref_x


def f16b(v):
    return {0.0: 0x0000, 0.5: 0x3800, 1.0: 0x3C00, 2.0: 0x4000}[v].to_bytes(2, "little")


def test_f16_decoder_matches_known_values():  # quant/mod.rs:921-928
    assert O.f16_to_f32(0x0000) == 0.0
    assert O.f16_to_f32(0x3800) == 0.5
    assert O.f16_to_f32(0x3C00) == 1.0
    assert O.f16_to_f32(0x4000) == 2.0
    assert O.f16_to_f32(0xC000) == -2.0


def test_f16_decoder_matches_ieee_half_exhaustively():
    # every finite pattern and the infinities against numpy's IEEE half
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    raw = h.astype("<u2").view(np.uint8)
    got = O.dequantize(O.F16, raw, 65536, checked=False)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    nan = np.isnan(want)
    assert np.isnan(got[nan]).all()
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_block_layouts_are_correct():  # quant/mod.rs:930-942
    assert O.block_layout(O.Q8_0) == (32, 34)
    assert O.block_layout(O.Q4_0) == (32, 18)
    assert O.block_layout(O.F16) == (1, 2)
    assert O.block_layout(O.Q2_K) == (256, 84)
    assert O.block_layout(O.Q3_K) == (256, 110)
    assert O.block_layout(O.Q4_K) == (256, 144)
    assert O.block_layout(O.Q5_K) == (256, 176)
    assert O.block_layout(O.Q6_K) == (256, 210)
    assert O.block_layout(3) is None
    assert O.block_layout(9) is None


def test_q5_k_adds_the_high_bit_from_qh():  # quant/mod.rs:944-958
    raw = bytearray(176)
    raw[0:2] = f16b(1.0)
    raw[2:4] = f16b(0.0)
    raw[4] = 1
    raw[16] = 0x01
    raw[48] = 0x03
    y = O.dequantize(O.Q5_K, np.frombuffer(bytes(raw), np.uint8), 256)
    assert y[0] == 19.0 and y[1] == 0.0


def test_q2_k_reads_2bit_quants_scaled_by_the_4bit_subscale():  # quant/mod.rs:960-973
    raw = bytearray(84)
    raw[0] = 0x02
    raw[16] = 0x03
    raw[80:82] = f16b(1.0)
    raw[82:84] = f16b(0.0)
    y = O.dequantize(O.Q2_K, np.frombuffer(bytes(raw), np.uint8), 256)
    assert y[0] == 6.0 and y[1] == 0.0


def test_q6_k_assembles_6bit_quants_centred_at_32():  # quant/mod.rs:975-991
    raw = bytearray(210)
    for i in range(192, 208):
        raw[i] = 1
    raw[208:210] = f16b(1.0)
    raw[0] = 0x05
    y = O.dequantize(O.Q6_K, np.frombuffer(bytes(raw), np.uint8), 256)
    assert y[0] == -27.0
    assert (y[1:] == -32.0).all()


def test_q4_k_reads_nibbles_scaled_by_the_subblock_scale():  # quant/mod.rs:993-1007
    raw = bytearray(144)
    raw[0:2] = f16b(1.0)
    raw[2:4] = f16b(0.0)
    raw[4] = 1
    raw[5] = 1
    raw[16] = 0x30
    y = O.dequantize(O.Q4_K, np.frombuffer(bytes(raw), np.uint8), 256)
    assert y[0] == 0.0 and y[32] == 3.0


def test_q8_0_dequantises_to_scale_times_q():  # quant/mod.rs:1009-1026
    qs = [0, 1, -2, 3] + [0] * 28
    raw = f16b(0.5) + bytes(q & 0xFF for q in qs)
    y = O.dequantize(O.Q8_0, np.frombuffer(raw, np.uint8), 32)
    assert list(y[:4]) == [0.0, 0.5, -1.0, 1.5]


def test_q4_0_uses_the_low_then_high_nibble_layout():  # quant/mod.rs:1028-1043
    qs = bytearray(16)
    qs[0] = 0x80
    qs[1] = 0x0F
    y = O.dequantize(O.Q4_0, np.frombuffer(f16b(1.0) + bytes(qs), np.uint8), 32)
    assert y[0] == -8.0 and y[16] == 0.0 and y[1] == 7.0 and y[17] == -8.0


def test_q8_0_round_trips_within_quantisation_error():  # quant/mod.rs:1045-1068
    orig = (np.arange(32, dtype=np.float32) - np.float32(16.0)) * np.float32(0.37)
    amax = np.float32(np.abs(orig).max())
    scale = np.float32(amax / np.float32(127.0))
    h = half_bits(scale)
    raw = h.to_bytes(2, "little")
    dec = O.f16_to_f32(h)
    q = np.clip(np.round(orig / scale), -127, 127).astype(np.int8)  # numpy rounds half even; no halves here
    raw += q.tobytes()
    y = O.dequantize(O.Q8_0, np.frombuffer(raw, np.uint8), 32)
    assert (np.abs(orig - y) <= dec + 1e-4).all()


def test_wrong_length_and_unsupported_type_are_errors():  # quant/mod.rs:1070-1076
    with pytest.raises(ValueError):
        O.dequantize(O.Q8_0, np.zeros(10, np.uint8), 32)
    with pytest.raises(ValueError):
        O.dequantize(O.Q4_K, np.zeros(100, np.uint8), 32)
    with pytest.raises(ValueError):
        O.dequantize(3, np.zeros(100, np.uint8), 32)
    with pytest.raises(ValueError):
        O.byte_size(O.Q8_0, 33)


def pack_scale_min_k4(scales, mins):  # quant/mod.rs:1107-1115
    s = [0] * 12
    for i in range(4):
        s[i] = (scales[i] & 0x3F) | ((scales[4 + i] >> 4) << 6)
        s[4 + i] = (mins[i] & 0x3F) | ((mins[4 + i] >> 4) << 6)
        s[8 + i] = (scales[4 + i] & 0x0F) | ((mins[4 + i] & 0x0F) << 4)
    return bytes(s)


def test_pack_scale_min_k4_round_trips_through_the_real_unpacker():  # quant/mod.rs:1117-1127
    import ctypes as C
    scales = [1, 5, 9, 13, 17, 21, 25, 29]
    mins = [2, 6, 10, 14, 18, 22, 26, 30]
    packed = (C.c_uint8 * 12)(*pack_scale_min_k4(scales, mins))
    for j in range(8):
        sc, m = C.c_uint8(), C.c_uint8()
        O.lib().or_get_scale_min_k4(j, packed, C.byref(sc), C.byref(m))
        assert (sc.value, m.value) == (scales[j], mins[j])


@pytest.mark.parametrize("qtype", O.INT8_TYPES)
def test_every_int8_kernel_matches_the_dequantise_then_dot_reference(qtype):  # quant/mod.rs:1184-1232
    elems, nbytes = O.block_layout(qtype)
    rows, bpr = 5, 3
    cols = bpr * elems
    rng = SplitMix(0xBEEF + qtype)
    weight = np.frombuffer(b"".join(random_block(qtype, rng) for _ in range(rows * bpr)), np.uint8)
    x = ref_x(rng, cols, 5)
    got = O.matvec(qtype, weight, rows, cols, x)
    for r in range(rows):
        row = weight[r * bpr * nbytes:(r + 1) * bpr * nbytes]
        deq = O.dequantize(qtype, row, cols)
        want = np.float32(O.dot(deq, x))
        step = max(np.float32(np.abs(x[i:i + 32]).max()) / np.float32(127.0) for i in range(0, cols, 32))
        tol = np.float32(np.abs(deq).sum()) * np.float32(step) * np.float32(0.5) + np.float32(1e-3)
        assert abs(got[r] - want) < tol


@pytest.mark.parametrize("qtype", O.INT8_TYPES)
def test_every_int8_kernel_reconstructs_weights_exactly_under_a_unit_activation(qtype):  # :1237-1266
    elems, nbytes = O.block_layout(qtype)
    cols = elems * 2
    rng = SplitMix(0x5EED + qtype)
    weight = np.frombuffer(random_block(qtype, rng) + random_block(qtype, rng), np.uint8)
    got = O.matvec(qtype, weight, 1, cols, np.ones(cols, np.float32))[0]
    deq = O.dequantize(qtype, weight[:nbytes * 2], cols)
    want = np.float32(0.0)
    for v in deq:
        want = np.float32(want + v)
    tol = abs(want) * 1e-4 + 1e-3
    assert abs(got - want) < tol


@pytest.mark.parametrize("qtype", O.INT8_TYPES)
def test_every_int8_kernel_handles_an_all_zero_row(qtype):  # quant/mod.rs:1268-1284
    elems, nbytes = O.block_layout(qtype)
    out = O.matvec(qtype, np.zeros(nbytes * 2, np.uint8), 1, elems * 2, np.full(elems * 2, 0.5, np.float32))
    assert np.isfinite(out[0])


@pytest.mark.parametrize("qtype", O.ALL_TYPES)
def test_matmul_agrees_with_repeated_matvec_for_every_supported_type(qtype):  # :1289-1319
    elems, _ = O.block_layout(qtype)
    cols = 256 if elems == 1 else elems * 2
    rows, n = 7, 5
    rng = SplitMix(0xC0FFEE + qtype)
    weight = random_rows(qtype, rows, cols, rng)
    xs = ref_x(rng, n * cols, 3)
    batched = O.matmul(qtype, weight, rows, cols, xs, n)
    for b in range(n):
        single = O.matvec(qtype, weight, rows, cols, xs[b * cols:(b + 1) * cols])
        assert np.array_equal(batched[b * rows:(b + 1) * rows].view(np.uint32), single.view(np.uint32))


def test_matmul_of_one_vector_is_matvec_and_bad_shapes_are_refused():  # :1321-1336
    rng = SplitMix(5)
    rows, cols = 4, 256
    weight = random_rows(O.Q6_K, rows, cols, rng)
    x = np.sin(np.arange(cols, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    a = O.matmul(O.Q6_K, weight, rows, cols, x, 1)
    b = O.matvec(O.Q6_K, weight, rows, cols, x)
    assert np.array_equal(a, b)
    with pytest.raises(ValueError):
        O.matmul(O.Q6_K, weight[:-1], rows, cols, x, 1)


def test_q3_k_closed_form():
    """Q3_K has no known-answer test in the reference; pin it by building blocks whose
    every field is chosen, and computing each weight from the ggml format definition:
    w = d * (sc - 32) * (q - 4*(1 - hbit)), element e of sub-block s=e//16, with the
    2-bit field at bits 2*j of qs[32*h + (e % 32)] and the high bit at bit 4*h + j of
    hmask[e % 32], where h = e // 128 and j = (e % 128) // 32."""
    rng = np.random.default_rng(7)
    for trial in range(20):
        sc6 = rng.integers(0, 64, 16)          # stored 6-bit scales (offset 32)
        low = rng.integers(0, 4, 256)
        hb = rng.integers(0, 2, 256)
        b = bytearray(110)
        for e in range(256):
            h, r = divmod(e, 128)
            j, l = divmod(r, 32)
            b[32 + 32 * h + l] |= int(low[e]) << (2 * j)
            if hb[e]:
                b[l] |= 1 << (4 * h + j)
        for i in range(4):  # the documented packing of 16 six-bit scales into 12 bytes
            b[96 + i] = (sc6[i] & 15) | ((sc6[8 + i] & 15) << 4)
            b[100 + i] = (sc6[4 + i] & 15) | ((sc6[12 + i] & 15) << 4)
            b[104 + i] = (sc6[i] >> 4) | ((sc6[4 + i] >> 4) << 2) | ((sc6[8 + i] >> 4) << 4) | ((sc6[12 + i] >> 4) << 6)
        d = np.float16(0.03125 * (trial + 1))
        b[108:110] = struct.pack("<e", float(d))
        got = O.dequantize(O.Q3_K, np.frombuffer(bytes(b), np.uint8), 256)
        q = low - 4 * (1 - hb)
        s = (sc6 - 32)[np.arange(256) // 16]
        want = (np.float32(d) * s.astype(np.float32)) * q.astype(np.float32)
        assert np.array_equal(got, want.astype(np.float32))


def test_quantize_activation_closed_form():
    """quant/mod.rs:331-345: each 32-block scales by amax/127 and rounds half away from
    zero; a block whose values are exact multiples of the step round-trips exactly."""
    x = np.zeros(64, np.float32)
    x[:32] = np.arange(-16, 16, dtype=np.float32) * np.float32(0.5)   # amax 8, step 8/127
    x[32] = 127.0
    x[33] = 63.5                                                        # exactly half a step
    x[34] = -63.5
    q, s = O.quantize_activation(x)
    assert s[0] == np.float32(8.0) / np.float32(127.0)
    assert s[1] == np.float32(1.0)
    assert q[32] == 127 and q[33] == 64 and q[34] == -64              # half away from zero
    assert q[40] == 0
    sums = O.block_sums(q, 16)
    assert sums[2] == int(q[32:48].astype(np.int32).sum())
    z, zs = O.quantize_activation(np.zeros(32, np.float32))
    assert (z == 0).all() and zs[0] == 0.0
