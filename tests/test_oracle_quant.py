"""Pins the oracle's f16 conversion and Q2/Q4/A8 block codecs.

Checks: numpy's binary16 (an independent IEEE implementation) for every
f16 bit pattern and for f32 rounding cases; the reference round-trip bounds
(Q/src/quant.rs:211-257); closed-form code tables; exhaustive unpack of
every byte value at every nibble/crumb position.
"""
import math

import numpy as np
import pytest


def test_f16_widening_matches_numpy_for_every_bit_pattern(orc):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))


def test_f16_narrowing_is_round_to_nearest_even(orc):
    rng = np.random.default_rng(7)
    xs = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-9, 5, 4000),
        # exact halfway points between neighbouring f16 values (ties to even)
        (np.arange(1, 2000, dtype=np.float32) + 0.5) / 1024.0,
        (np.arange(1, 500, dtype=np.float32) + 0.5) * 2.0 ** -24,  # subnormal ties
        np.array([65504.0, 65519.0, 65520.0, 1e6, -1e6, 0.0, -0.0, 2.0 ** -25, 2.0 ** -26], dtype=np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):  # 65520 and 1e6 round to infinity on purpose
        ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got, ref)


def _fixture():
    # Q/src/quant.rs:211-213
    return np.array([math.sin((i - 31.5) / 31.5) for i in range(64)], dtype=np.float32)


def test_q2_round_trip_bound_and_determinism(orc):
    blk = orc.q2_quantize(_fixture())
    assert len(blk) == 18
    assert orc.q2_quantize(_fixture()) == blk
    deq = np.array([orc.q2_value(blk, i) for i in range(64)])
    assert np.all(np.abs(deq - _fixture()) <= 0.34)  # Q/src/quant.rs:215-225


def test_q4_round_trip_bound_and_determinism(orc):
    blk = orc.q4_quantize(_fixture())
    assert len(blk) == 34
    deq = np.array([orc.q4_value(blk, i) for i in range(64)])
    assert np.all(np.abs(deq - _fixture()) <= 0.07)  # Q/src/quant.rs:227-237


def test_quantize_rejects_non_finite(orc):
    v = _fixture()
    v[3] = np.nan
    with pytest.raises(orc.OracleError) as e:
        orc.q2_quantize(v)
    assert e.value.code == 3  # InvalidArtifact


def test_a8_extreme_codes_and_bound(orc):
    # Q/src/quant.rs:246-257
    scale, codes = orc.a8_quantize(_fixture())
    assert codes[0] == -127 and codes[63] == 127
    deq = scale * codes.astype(np.float32)
    assert np.all(np.abs(deq - _fixture()) <= scale * 0.501)
    s0, c0 = orc.a8_quantize(np.zeros(64, np.float32))
    assert s0 == 0.0 and not c0.any()


def test_zero_block_has_zero_scale(orc):
    assert orc.q4_quantize(np.zeros(64, np.float32)) == bytes(34)
    assert orc.q2_quantize(np.zeros(64, np.float32)) == bytes(18)


def _block(scale_bits: int, body: bytes) -> bytes:
    return bytes([scale_bits & 0xFF, scale_bits >> 8]) + body


def test_q4_unpack_exhaustive_every_byte_value(orc):
    # scale 1.0: value = (c - 7.5)/7.5 with c the low (even i) or high (odd i) nibble
    one = 0x3C00
    for byte in range(256):
        blk = _block(one, bytes([byte]) * 32)
        lo, hi = byte & 0xF, byte >> 4
        for i in (0, 1, 62, 63):
            c = lo if i % 2 == 0 else hi
            want = np.float32(np.float32(c) - np.float32(7.5)) / np.float32(7.5)
            assert orc.q4_value(blk, i) == want


def test_q2_unpack_exhaustive_every_byte_value(orc):
    one = 0x3C00
    table = {0: -1.0, 1: float(np.float32(-1.0) / np.float32(3.0)), 2: float(np.float32(1.0) / np.float32(3.0)),
             3: 1.0}
    for byte in range(256):
        blk = _block(one, bytes([byte]) * 16)
        for i in range(8):
            c = (byte >> (2 * (i % 4))) & 3
            assert orc.q2_value(blk, i) == np.float32(table[c])


def test_q4_code_table_is_sixteen_uniform_levels(orc):
    # Closed form: codes 0 and 15 are -1 and +1, spacing 2/15, midpoint between 7 and 8.
    one = 0x3C00
    vals = [orc.q4_value(_block(one, bytes([c | (c << 4)]) * 32), 0) for c in range(16)]
    assert vals[0] == -1.0 and vals[15] == 1.0
    assert np.allclose(np.diff(vals), 2.0 / 15.0, atol=1e-7)
    assert abs(vals[7] + vals[8]) < 1e-7
