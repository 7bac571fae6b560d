"""Pins the oracle's fused matvec (scalar verifier and AVX2 profile).

Ports the crate's own CPU tests (Q/src/backend/cpu.rs:732-1126) and the
loader closed form (Q/src/loader.rs:460-543), and bounds the scalar oracle
by an f64 brute force over the dequantized matrix (a dropped term, a wrong
nibble or a transposed operand fails it).
"""
import json
import math
import os

import numpy as np
import pytest

import ctox_hip.synth as synth

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "crate_goldens.json")))
SIMD_TOLERANCE = 2e-4  # Q/src/backend/cpu.rs:745


def encode_fixture(orc, dtype, rows, cols, amp=0.75):
    # Q/src/backend/cpu.rs:751-769
    out = bytearray()
    for mb in range(rows * cols // 64):
        vals = np.array([math.sin(np.float32(mb * 64 + i) * np.float32(0.013579)) * amp for i in range(64)],
                        dtype=np.float32)
        out += orc.q2_quantize(vals) if dtype == 0 else orc.q4_quantize(vals)
    return bytes(out)


def fused_case(orc, dtype, rows, cols, act):
    # Q/src/backend/cpu.rs:774-812
    w = encode_fixture(orc, dtype, rows, cols)
    x = np.array([math.cos(i * 0.03125) for i in range(cols)], np.float32)
    s_in = np.array([0.75 + 0.005 * (i % 7) for i in range(cols)], np.float32)
    s_out = np.array([1.25 - 0.05 * (r % 5) for r in range(rows)], np.float32)
    bias = np.array([math.sin(r * 1.7) * 0.1 for r in range(rows)], np.float32)
    mv = orc.MatVec(dtype, w, rows, cols, x, ("f32", s_in), ("f32", s_out), bias, act)
    return mv.run(orc.SCALAR), (mv.run(orc.AVX2) if orc.avx2_available() else mv.run(orc.SCALAR))


@pytest.mark.parametrize("dtype,rows,cols,act", [(0, 7, 192, 1), (1, 7, 192, 1), (0, 3, 64, 0), (1, 3, 64, 0)])
def test_simd_matches_scalar(orc, dtype, rows, cols, act):
    scalar, simd = fused_case(orc, dtype, rows, cols, act)
    assert np.all(np.abs(scalar - simd) <= SIMD_TOLERANCE)


def test_packed_f16_scales_match_f32_scales(orc):
    # Q/src/backend/cpu.rs:834-875
    w = encode_fixture(orc, 0, 2, 64)
    x = np.array([math.sin(i * 0.0625) for i in range(64)], np.float32)
    s_in = np.array([np.float16(0.75 + (i % 9) * 0.03125) for i in range(64)], np.float32)
    s_out = np.array([np.float16(1.25), np.float16(0.875)], np.float32)
    f16in = s_in.astype(np.float16).view(np.uint8)
    f16out = s_out.astype(np.float16).view(np.uint8)
    for prof in (orc.SCALAR, orc.AVX2):
        a = orc.fused_matvec(0, w, 2, 64, x, ("f32", s_in), ("f32", s_out), profile=prof)
        b = orc.fused_matvec(0, w, 2, 64, x, ("f16le", f16in), ("f16le", f16out), profile=prof)
        assert np.array_equal(a, b)


def test_mixed_rows_equal_their_pure_kernels(orc):
    # Q/src/backend/cpu.rs:877-952
    cols = 128
    q2 = encode_fixture(orc, 0, 2, cols)
    q4 = encode_fixture(orc, 1, 2, cols)
    x = np.array([math.cos(i * 0.0234375) for i in range(cols)], np.float32)
    segs = [(0, 0, 2, 0, 0, len(q2)), (1, 2, 4, 1, len(q2), len(q4))]
    for prof in (orc.SCALAR, orc.AVX2):
        mixed = orc.fused_matvec(2, q2 + q4, 4, cols, x, segments=segs, profile=prof)
        assert np.array_equal(mixed[:2], orc.fused_matvec(0, q2, 2, cols, x, profile=prof))
        assert np.array_equal(mixed[2:], orc.fused_matvec(1, q4, 2, cols, x, profile=prof))


def test_fanout_equals_independent(orc):
    # Q/src/backend/cpu.rs:954-1010
    x = np.array([math.sin(i * 0.0625) for i in range(64)], np.float32)
    q2 = encode_fixture(orc, 0, 2, 64)
    q4 = encode_fixture(orc, 1, 3, 64)
    shared = np.full(64, 1.125, np.float32)
    a = orc.MatVec(0, q2, 2, 64, x, ("f32", shared))
    b = orc.MatVec(1, q4, 3, 64, x, ("f32", shared))
    outs = orc.fanout([a, b], orc.AVX2)
    assert np.array_equal(outs[0], a.run(orc.AVX2)) and np.array_equal(outs[1], b.run(orc.AVX2))
    with pytest.raises(orc.OracleError) as e:
        orc.fanout([], orc.AVX2)


def test_mixed_rejects_non_contiguous_segments(orc):
    # Q/src/backend/cpu.rs:1012-1042
    w = encode_fixture(orc, 0, 2, 64)
    with pytest.raises(orc.OracleError) as e:
        orc.fused_matvec(2, w, 2, 64, np.ones(64, np.float32), segments=[(0, 1, 2, 0, 0, len(w))])
    assert e.value.code == 3


@pytest.mark.parametrize("dtype,mul,add,scale", [(0, 0x45, 0x1B, 0.625), (1, 0x9E, 0x3D, 0.375)])
def test_packed_dot_decodes_arbitrary_codes(orc, dtype, mul, add, scale):
    # Q/src/backend/cpu.rs:1044-1088
    n = 16 if dtype == 0 else 32
    codes = bytes(((i * mul) + add) & 0xFF for i in range(n))
    if dtype == 0:
        x = np.array([math.sin(i * 0.11) + 0.25 for i in range(64)], np.float32)
    else:
        x = np.array([math.cos(i * 0.07) - 0.125 for i in range(64)], np.float32)
    hb = orc.f32_to_f16(scale)
    blk = bytes([hb & 0xFF, hb >> 8]) + codes
    val = orc.q2_value if dtype == 0 else orc.q4_value
    ref = np.float32(0.0)
    for i in range(64):
        ref = np.float32(ref + np.float32(val(blk, i)) * x[i])
    for prof in (orc.SCALAR, orc.AVX2):
        assert abs(ref - orc.packed_dot(dtype, prof, orc.f16_to_f32(hb), codes, x)) <= 1e-5


def test_loader_closed_form(orc):
    # Q/src/loader.rs:460-543: a Q2 block of 0.5 with s_out 1.5 -> 48.0; row -> 0.75
    g = GOLD["loader_closed_form"]
    blk = orc.q2_quantize(np.full(64, 0.5, np.float32))
    s_in = np.ones(64, np.float16).view(np.uint8)
    s_out = np.array([1.5], np.float16).view(np.uint8)
    y = orc.fused_matvec(0, blk, 1, 64, np.ones(64, np.float32), ("f16le", s_in), ("f16le", s_out))
    assert abs(y[0] - g["matvec"]) < g["tol"]
    row = orc.recovered_row(0, blk, 64, ("f16le", s_in), 1.5)
    assert np.all(np.abs(row - g["embedding"]) < g["tol"])


@pytest.mark.parametrize("dtype", [0, 1])
def test_scalar_oracle_matches_f64_brute_force(orc, dtype):
    rows, cols = 37, 1024
    w = synth.random_matrix(dtype, rows, cols, seed=11)
    x = synth.activation("normal", cols, seed=12)[0]
    rng = np.random.default_rng(13)
    s_in = rng.uniform(0.75, 1.25, cols).astype(np.float16)
    s_out = rng.uniform(0.75, 1.25, rows).astype(np.float16)
    bias = rng.standard_normal(rows).astype(np.float32) * 0.1
    dense = synth.unpack_dense(dtype, w, rows, cols)
    ref = ((dense @ (x.astype(np.float64) * s_in.astype(np.float64))) + bias) * s_out.astype(np.float64)
    ref = ref / (1.0 + np.exp(-ref))
    got = orc.fused_matvec(dtype, w, rows, cols, x, ("f16le", s_in.view(np.uint8)),
                           ("f16le", s_out.view(np.uint8)), bias, 1)
    scale = np.sqrt(np.mean(ref ** 2))
    assert np.max(np.abs(got - ref)) <= 1e-5 * scale + 1e-7


def test_validation_errors_match_crate(orc):
    w = encode_fixture(orc, 1, 2, 64)
    x = np.ones(64, np.float32)
    cases = [
        (dict(columns=65), 7),             # columns not a multiple of 64
        (dict(rows=0), 7),
        (dict(weights=w[:-1]), 7),         # short weight buffer
        (dict(dtype=3), 4),                # F16 is not a quantized matvec dtype
        (dict(segments=[(0, 0, 2, 1, 0, len(w))]), 3),  # pure op with segments
        (dict(dtype=2), 3),                # mixed without segments
    ]
    for over, code in cases:
        args = dict(dtype=1, weights=w, rows=2, columns=64, input=x)
        args.update(over)
        inp = args.pop("input")
        if args["columns"] != 64:
            inp = np.ones(args["columns"], np.float32)
        with pytest.raises(orc.OracleError) as e:
            orc.fused_matvec(args["dtype"], args["weights"], args["rows"], args["columns"], inp,
                             segments=args.get("segments", ()))
        assert e.value.code == code, over
    bad = bytearray(w)
    bad[0], bad[1] = 0x00, 0x7C  # +inf scale
    with pytest.raises(orc.OracleError) as e:
        orc.fused_matvec(1, bytes(bad), 2, 64, x)
    assert e.value.code == 3
