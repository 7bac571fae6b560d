"""GPU parity of the fused Q2/Q4 matvec and its small-M verify variant
against the C oracle (scalar verifier of Q/src/backend/cpu.rs:558-575).

Tolerance (stated per the BASELINE north star): elementwise
|gpu - oracle| <= 1e-3 * (|oracle| + rms(oracle)). The int8-MFMA kernel is
exact in its integer part, so the observed error is ~1e-6 relative; the
tests also assert a normwise bound of 2e-5 to catch regressions early.
Unpacking and indexing are bit-exact by construction and are additionally
checked by the recovered-row kernels, which must match the oracle exactly.
"""
import math
import sys

import numpy as np
import pytest

import ctox_hip
import ctox_hip.synth as synth

pytestmark = pytest.mark.gpu

RTOL = 1e-3
NORMWISE = 2e-5


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def check(got, ref, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    rms = math.sqrt(float(np.mean(ref ** 2))) if ref.size else 0.0
    d = np.abs(got - ref)
    assert np.all(d <= RTOL * (np.abs(ref) + rms) + 1e-30), f"{what}: max elementwise {d.max()} (rms {rms})"
    norm = d.max() / max(np.abs(ref).max(), 1e-30)
    assert norm <= NORMWISE, f"{what}: normwise {norm}"
    return norm


def make_case(dtype, rows, cols, seed, s_kind="f16", bias=True, act=ctox_hip.Activation.Identity, batch=1,
              xkind="normal"):
    w = synth.random_matrix(dtype, rows, cols, seed)
    x = synth.activation(xkind, cols, seed + 1, batch)
    rng = np.random.default_rng(seed + 2)
    s_in = rng.uniform(0.75, 1.25, cols).astype(np.float32)
    s_out = rng.uniform(0.75, 1.25, rows).astype(np.float32)
    b = (rng.standard_normal(rows) * 0.05).astype(np.float32) if bias else None
    if s_kind == "f16":
        si = ctox_hip.ScaleSlice.F16Le(s_in.astype(np.float16).view(np.uint8))
        so = ctox_hip.ScaleSlice.F16Le(s_out.astype(np.float16).view(np.uint8))
        osi, oso = ("f16le", s_in.astype(np.float16).view(np.uint8)), ("f16le", s_out.astype(np.float16).view(np.uint8))
    elif s_kind == "f32":
        si, so = ctox_hip.ScaleSlice.F32(s_in), ctox_hip.ScaleSlice.F32(s_out)
        osi, oso = ("f32", s_in), ("f32", s_out)
    else:
        si = so = osi = oso = None
    op = ctox_hip.FusedMatVec(ctox_hip.TensorDType(dtype), w, rows, cols, x[0], s_in=si, s_out=so, bias=b,
                              activation=act)
    return op, (w, x, osi, oso, b)


def oracle_rows(orc, dtype, rows, cols, parts, act, segments=()):
    w, x, osi, oso, b = parts
    return np.stack([orc.fused_matvec(dtype, w, rows, cols, x[m], osi, oso, b, int(act), segments)
                     for m in range(x.shape[0])])


SMALL = [(1, 64), (3, 64), (7, 192), (65, 128), (64, 1024), (100, 1088), (257, 2112), (130, 5120)]


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("rows,cols", SMALL)
def test_matvec_host_api_small_shapes(hip, orc, dtype, rows, cols):
    say(f"case matvec dtype={dtype} rows={rows} cols={cols}")
    for i, (sk, bias, act) in enumerate([("f16", True, ctox_hip.Activation.Silu), ("f32", False, ctox_hip.Activation.Identity),
                                         ("none", True, ctox_hip.Activation.Identity)]):
        op, parts = make_case(dtype, rows, cols, 100 + rows + i, sk, bias, act)
        got = hip.fused_matvec(op)
        ref = oracle_rows(orc, dtype, rows, cols, parts, act)[0]
        check(got, ref, f"dtype={dtype} {rows}x{cols} {sk}")


# Raw launches on weights without a tiled copy run the crate-layout kernels:
# batch 1 on columns % 512 == 0 the slice kernels (28 (Q4) / 56 (Q2) blocks
# per slice, all slices requested up front for 1..3 slices, walked beyond),
# M = 2..8 the small-M slice kernels. These widths give every slice count of
# both dtypes at least once.
SLICE_COLS = [512, 1536, 3584, 5120, 7168, 10752, 17408]


def raw_run(hip, dtype, parts, rows, cols, act):
    """ctox_hip_launch_fused_matvec on unregistered device weights (f16 scales)."""
    torch = _torch()
    w, x, osi, oso, b = parts
    dw = torch.from_numpy(np.ascontiguousarray(w)).cuda()
    dx = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    dsi = torch.from_numpy(np.ascontiguousarray(osi[1]).view(np.int16)).cuda()
    dso = torch.from_numpy(np.ascontiguousarray(oso[1]).view(np.int16)).cuda()
    db = torch.from_numpy(b).cuda() if b is not None else None
    dy = torch.empty((x.shape[0], rows), device="cuda")
    hip.launch_fused_matvec(ctox_hip.TensorDType(dtype), dw.data_ptr(), dx.data_ptr(), dsi.data_ptr(), dso.data_ptr(),
                            None if db is None else db.data_ptr(), dy.data_ptr(), rows, cols, act, x.shape[0],
                            torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return dy.cpu().numpy()


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("cols", SLICE_COLS)
def test_batch1_slice_counts(hip, orc, dtype, cols):
    for rows in (16, 37):
        say(f"case slices dtype={dtype} rows={rows} cols={cols}")
        op, parts = make_case(dtype, rows, cols, 7 * cols + rows, "f16", True, ctox_hip.Activation.Silu)
        got = raw_run(hip, dtype, parts, rows, cols, ctox_hip.Activation.Silu)[0]
        ref = oracle_rows(orc, dtype, rows, cols, parts, ctox_hip.Activation.Silu)[0]
        check(got, ref, f"slices dtype={dtype} {rows}x{cols}")


def test_crate_fixture_cases(hip, orc):
    # Q/src/backend/cpu.rs:774-832 fixtures (sin weights, cos input, f32 scales, bias, SiLU)
    from test_oracle_matvec import encode_fixture
    for dtype, rows, cols, act in [(0, 7, 192, 1), (1, 7, 192, 1), (0, 3, 64, 0), (1, 3, 64, 0)]:
        say(f"case crate fixture dtype={dtype} rows={rows} cols={cols}")
        w = encode_fixture(orc, dtype, rows, cols)
        x = np.array([math.cos(i * 0.03125) for i in range(cols)], np.float32)
        s_in = np.array([0.75 + 0.005 * (i % 7) for i in range(cols)], np.float32)
        s_out = np.array([1.25 - 0.05 * (r % 5) for r in range(rows)], np.float32)
        bias = np.array([math.sin(r * 1.7) * 0.1 for r in range(rows)], np.float32)
        ref = orc.fused_matvec(dtype, w, rows, cols, x, ("f32", s_in), ("f32", s_out), bias, act)
        got = hip.fused_matvec(ctox_hip.FusedMatVec(ctox_hip.TensorDType(dtype), np.frombuffer(w, np.uint8), rows,
                                                    cols, x, s_in=ctox_hip.ScaleSlice.F32(s_in),
                                                    s_out=ctox_hip.ScaleSlice.F32(s_out), bias=bias,
                                                    activation=ctox_hip.Activation(act)))
        assert np.all(np.abs(got - ref) <= 2e-4)  # the crate's SIMD tolerance, Q/src/backend/cpu.rs:745
        check(got, ref, "crate fixture")


def test_loader_closed_form_on_gpu(hip, orc):
    # Q/src/loader.rs:460-543: a Q2 block of 0.5, s_in 1, s_out 1.5 -> 48.0; embedding row -> 0.75
    blk = np.frombuffer(orc.q2_quantize(np.full(64, 0.5, np.float32)), np.uint8)
    s_in = ctox_hip.ScaleSlice.F16Le(np.ones(64, np.float16).view(np.uint8))
    s_out = ctox_hip.ScaleSlice.F16Le(np.array([1.5], np.float16).view(np.uint8))
    y = hip.fused_matvec(ctox_hip.FusedMatVec(ctox_hip.TensorDType.Q2B64, blk, 1, 64, np.ones(64, np.float32),
                                              s_in=s_in, s_out=s_out))
    assert abs(y[0] - 48.0) < 1e-6
    row = hip.recovered_row(ctox_hip.RecoveredRow(ctox_hip.TensorDType.Q2B64, blk, 64, s_in, 1.5))
    assert np.all(np.abs(row - 0.75) < 1e-6)


def _torch():
    import torch
    assert torch.cuda.is_available()
    return torch


def resident_run(hip, op, xs):
    """Prepare the matrix in HBM and dispatch a [batch, cols] activation."""
    torch = _torch()
    m = hip.prepare(op)
    dx = torch.from_numpy(np.ascontiguousarray(xs)).cuda()
    dy = torch.empty((xs.shape[0], op.rows), dtype=torch.float32, device="cuda")
    m.dispatch(dx.data_ptr(), xs.shape[0], dy.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = dy.cpu().numpy()
    m.close()
    return out


@pytest.mark.parametrize("cfg", ["config1_q4_up_17408x5120", "config2_q2_down_5120x17408"])
def test_baseline_full_shapes(hip, orc, cfg):
    dtype, rows, cols, xkind = (1, 17408, 5120, "normal") if cfg.startswith("config1") else (0, 5120, 17408, "swiglu")
    for sk in ("none", "f16"):
        say(f"case {cfg} scales={sk}")
        op, parts = make_case(dtype, rows, cols, 7, sk, bias=False, xkind=xkind)
        got = resident_run(hip, op, parts[1])
        ref = oracle_rows(orc, dtype, rows, cols, parts, ctox_hip.Activation.Identity)
        n = check(got, ref, cfg)
        say(f"  normwise rel err {n:.3e}")



@pytest.mark.parametrize("mode", ["1", "0"])
def test_tiled_combine_modes(orc, mode, monkeypatch):
    """Both ways the tiled kernels' chunks meet give the oracle's
    rows: by arrival (the last chunk to arrive for a tile adds them, used for
    launches larger than the device holds at once) and by the last chunk's
    waves (used when every workgroup is resident). CTOX_ARRIVE forces one
    of them for a backend of this test's own; the 151936-row LM-head shape
    takes the arrival path by itself."""
    import ctox_hip
    monkeypatch.setenv("CTOX_ARRIVE", mode)
    hip2 = ctox_hip.HipBackend(0)
    try:
        for dtype, rows, cols, xkind in ((1, 17408, 5120, "normal"), (0, 5120, 17408, "swiglu"),
                                         (1, 4096 + 48, 1024, "normal")):
            say(f"case combine mode={mode} dtype={dtype} {rows}x{cols}")
            op, parts = make_case(dtype, rows, cols, 41, "f16", bias=False, xkind=xkind)
            for rep in range(2):  # the counts are back at zero for the next launch
                got = resident_run(hip2, op, parts[1])
                ref = oracle_rows(orc, dtype, rows, cols, parts, ctox_hip.Activation.Identity)
                check(got, ref, f"combine mode={mode} rep={rep}")
        for batch in (3, 8):  # the small-M kernels (one and two token groups)
            say(f"case combine mode={mode} small-m batch={batch}")
            op, parts = make_case(1, 17408, 5120, 45, "f16", bias=False, batch=batch)
            for rep in range(2):
                got = resident_run(hip2, op, parts[1])
                ref = oracle_rows(orc, 1, 17408, 5120, parts, ctox_hip.Activation.Identity)
                check(got, ref, f"combine mode={mode} batch={batch} rep={rep}")
    finally:
        hip2.close()
    monkeypatch.delenv("CTOX_ARRIVE")
    hip3 = ctox_hip.HipBackend(0)
    try:
        say("case combine default: LM-head shape 151936x5120")
        op, parts = make_case(1, 151936, 5120, 43, "f16", bias=False)
        got = resident_run(hip3, op, parts[1])
        ref = oracle_rows(orc, 1, 151936, 5120, parts, ctox_hip.Activation.Identity)
        check(got, ref, "LM head")
        del op, parts, got, ref
        # The largest single matrix of the crate's model: the LM head over its
        # 248320-token vocabulary (675 MB of Q4 rows), batch 1 and a 5-row verify.
        for batch in (1, 5):
            say(f"case combine default: crate LM head 248320x5120 batch={batch}")
            op, parts = make_case(1, 248320, 5120, 47, "f16", bias=False, batch=batch)
            got = resident_run(hip3, op, parts[1])
            ref = oracle_rows(orc, 1, 248320, 5120, parts, ctox_hip.Activation.Identity)
            check(got, ref, f"crate LM head batch={batch}")
            del op, parts, got, ref
    finally:
        hip3.close()

# One decoder layer (Q/src/tensor_contract.rs:70-240): q_proj 12288 (crate) / 6144 (BASELINE),
# k/v 1024, o 5120x6144, gate/up 17408x5120, down 5120x17408.
LAYER = [("q_proj_crate", 1, 12288, 5120), ("q_proj_baseline", 1, 6144, 5120), ("k_proj", 1, 1024, 5120),
         ("v_proj", 1, 1024, 5120), ("o_proj", 1, 5120, 6144), ("gate_proj", 1, 17408, 5120),
         ("up_proj", 1, 17408, 5120), ("down_proj_q2", 0, 5120, 17408)]


@pytest.mark.parametrize("batch", [2, 4, 5, 8])
def test_verify_small_m_layer_projections(hip, orc, batch):
    for name, dtype, rows, cols in LAYER:
        say(f"case verify batch={batch} {name} {rows}x{cols}")
        op, parts = make_case(dtype, rows, cols, 31 + rows, "f16", bias=False, batch=batch)
        got = resident_run(hip, op, parts[1])
        ref = oracle_rows(orc, dtype, rows, cols, parts, ctox_hip.Activation.Identity)
        check(got, ref, f"{name} batch={batch}")


@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 6, 7, 8])
def test_batched_ragged(hip, orc, batch):
    for dtype, rows, cols in [(0, 77, 192), (1, 77, 192), (1, 130, 2112)]:
        say(f"case ragged batch={batch} dtype={dtype} {rows}x{cols}")
        op, parts = make_case(dtype, rows, cols, 5 + batch, "f32", bias=True, act=ctox_hip.Activation.Silu,
                              batch=batch)
        got = resident_run(hip, op, parts[1])
        ref = oracle_rows(orc, dtype, rows, cols, parts, ctox_hip.Activation.Silu)
        check(got, ref, f"ragged batch={batch}")


@pytest.mark.parametrize("batch", [2, 3, 5, 8])
@pytest.mark.parametrize("dtype", [0, 1])
def test_small_m_slice_counts(hip, orc, batch, dtype):
    """M = 2..8 on columns % 512 == 0 runs the small-M slice kernels (28 / 26
    blocks per slice, partial last slices, rows not a multiple of 16)."""
    for cols in (512, 1664, 3584, 7168, 17408):
        rows = 37
        say(f"case small-m slices batch={batch} dtype={dtype} {rows}x{cols}")
        op, parts = make_case(dtype, rows, cols, 3 * cols + batch, "f16", bias=True, act=ctox_hip.Activation.Silu,
                              batch=batch)
        got = raw_run(hip, dtype, parts, rows, cols, ctox_hip.Activation.Silu)
        ref = oracle_rows(orc, dtype, rows, cols, parts, ctox_hip.Activation.Silu)
        check(got, ref, f"small-m slices batch={batch} dtype={dtype} {rows}x{cols}")


def test_mixed_segments_match_pure(hip, orc):
    say("case mixed segments")
    cols = 1088
    q2 = synth.random_matrix(0, 70, cols, 1)
    q4 = synth.random_matrix(1, 90, cols, 2)
    x = synth.activation("normal", cols, 3)[0]
    segs = [ctox_hip.QuantSegment(0, 0, 70, ctox_hip.TensorDType.Q2B64, 0, q2.size),
            ctox_hip.QuantSegment(1, 70, 160, ctox_hip.TensorDType.Q4B64, q2.size, q4.size)]
    mixed = hip.fused_matvec(ctox_hip.FusedMatVec(ctox_hip.TensorDType.MixedQ2Q4B64, np.concatenate([q2, q4]), 160,
                                                  cols, x, segments=segs))
    a = hip.fused_matvec(ctox_hip.FusedMatVec(ctox_hip.TensorDType.Q2B64, q2, 70, cols, x))
    b = hip.fused_matvec(ctox_hip.FusedMatVec(ctox_hip.TensorDType.Q4B64, q4, 90, cols, x))
    assert np.array_equal(mixed[:70], a) and np.array_equal(mixed[70:], b)
    ref = orc.fused_matvec(2, np.concatenate([q2, q4]).tobytes(), 160, cols, x,
                           segments=[(0, 0, 70, 0, 0, q2.size), (1, 70, 160, 1, q2.size, q4.size)])
    check(mixed, ref, "mixed")


def test_fanout_and_determinism(hip):
    say("case fanout/determinism")
    cols = 5120
    x = synth.activation("normal", cols, 4)[0]
    s_in = ctox_hip.ScaleSlice.F16Le(np.full(cols, 1.125, np.float16).view(np.uint8))
    ops = [ctox_hip.FusedMatVec(ctox_hip.TensorDType(d), synth.random_matrix(d, r, cols, 10 + r), r, cols, x,
                                s_in=s_in) for d, r in [(0, 200), (1, 300)]]
    outs = hip.fused_matvec_fanout(ops)
    for o, op in zip(outs, ops):
        assert np.array_equal(o, hip.fused_matvec(op))
        assert np.array_equal(hip.fused_matvec(op), hip.fused_matvec(op))
    with pytest.raises(ctox_hip.ShapeError):
        hip.fused_matvec_fanout([])


def test_device_fanout_equals_independent(hip):
    torch = _torch()
    say("case device fanout")
    cols = 5120
    x = synth.activation("normal", cols, 8, 3)
    s_in = ctox_hip.ScaleSlice.F16Le(np.linspace(0.8, 1.2, cols).astype(np.float16).view(np.uint8))
    mats = [hip.prepare(ctox_hip.FusedMatVec(ctox_hip.TensorDType(d), synth.random_matrix(d, r, cols, r), r, cols,
                                             s_in=s_in)) for d, r in [(1, 1024), (0, 640), (1, 48)]]
    dx = torch.from_numpy(x).cuda()
    outs = [torch.empty((3, m.rows), device="cuda") for m in mats]
    hip.dispatch_fanout(mats, dx.data_ptr(), 3, [o.data_ptr() for o in outs], torch.cuda.current_stream().cuda_stream)
    for m, o in zip(mats, outs):
        single = torch.empty_like(o)
        m.dispatch(dx.data_ptr(), 3, single.data_ptr(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(o, single)


def test_raw_launch_matches_resident_dispatch(hip):
    torch = _torch()
    say("case raw launch")
    rows, cols = 1000, 5120
    w = synth.random_matrix(1, rows, cols, 77)
    x = synth.activation("normal", cols, 78, 2)
    s_in = np.linspace(0.9, 1.1, cols).astype(np.float16)
    s_out = np.linspace(1.1, 0.9, rows).astype(np.float16)
    bias = np.linspace(-0.1, 0.1, rows).astype(np.float32)
    op = ctox_hip.FusedMatVec(ctox_hip.TensorDType.Q4B64, w, rows, cols, s_in=ctox_hip.ScaleSlice.F16Le(s_in.view(np.uint8)),
                              s_out=ctox_hip.ScaleSlice.F16Le(s_out.view(np.uint8)), bias=bias,
                              activation=ctox_hip.Activation.Silu)
    want = resident_run(hip, op, x)
    dw = torch.from_numpy(w).cuda()
    dx = torch.from_numpy(x).cuda()
    dsi = torch.from_numpy(s_in.view(np.int16)).cuda()
    dso = torch.from_numpy(s_out.view(np.int16)).cuda()
    db = torch.from_numpy(bias).cuda()
    dy = torch.empty((2, rows), device="cuda")
    hip.launch_fused_matvec(ctox_hip.TensorDType.Q4B64, dw.data_ptr(), dx.data_ptr(), dsi.data_ptr(), dso.data_ptr(),
                            db.data_ptr(), dy.data_ptr(), rows, cols, ctox_hip.Activation.Silu, 2,
                            torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    # The raw launch streams the crate-layout rows, the resident matrix its
    # tiled copy: the same sums in another order, both within tolerance of
    # the oracle.
    w_ref = oracle_rows(__import__("oracle.oracle", fromlist=["oracle"]), 1, rows, cols,
                        (w, x, ("f16le", s_in.view(np.uint8)), ("f16le", s_out.view(np.uint8)), bias),
                        ctox_hip.Activation.Silu)
    check(dy.cpu().numpy(), w_ref, "raw launch")
    check(want, w_ref, "resident dispatch")


def test_error_contract(hip):
    say("case errors")
    w = synth.random_matrix(1, 4, 128, 1)
    x = np.ones(128, np.float32)
    T = ctox_hip.TensorDType
    with pytest.raises(ctox_hip.ShapeError):
        hip.fused_matvec(ctox_hip.FusedMatVec(T.Q4B64, w[:-1], 4, 128, x))
    with pytest.raises(ctox_hip.ShapeError):
        hip.fused_matvec(ctox_hip.FusedMatVec(T.Q4B64, w, 4, 100, np.ones(100, np.float32)))
    with pytest.raises(ctox_hip.UnsupportedDType):
        hip.fused_matvec(ctox_hip.FusedMatVec(T.F16, w, 4, 128, x))
    with pytest.raises(ctox_hip.InvalidArtifact):
        hip.fused_matvec(ctox_hip.FusedMatVec(T.MixedQ2Q4B64, w, 4, 128, x))
    with pytest.raises(ctox_hip.InvalidArtifact):
        hip.fused_matvec(ctox_hip.FusedMatVec(T.MixedQ2Q4B64, w, 4, 128, x,
                                              segments=[ctox_hip.QuantSegment(0, 1, 4, T.Q4B64, 0, w.size)]))
    bad = w.copy()
    bad[0], bad[1] = 0x00, 0x7C
    with pytest.raises(ctox_hip.InvalidArtifact):
        hip.fused_matvec(ctox_hip.FusedMatVec(T.Q4B64, bad, 4, 128, x))
    nan_x = x.copy()
    nan_x[5] = np.nan
    with pytest.raises(ctox_hip.InvalidState):
        hip.fused_matvec(ctox_hip.FusedMatVec(T.Q4B64, w, 4, 128, nan_x))
    with pytest.raises(ctox_hip.ShapeError):
        m = hip.prepare(ctox_hip.FusedMatVec(T.Q4B64, w, 4, 128))
        m.dispatch(1, 9, 1)


@pytest.mark.parametrize("dtype", [0, 1])
def test_recovered_row_bit_exact(hip, orc, dtype):
    say(f"case recovered row dtype={dtype}")
    cols = 5120
    w = synth.random_matrix(dtype, 1, cols, 3 + dtype)
    s_in_f16 = np.random.default_rng(0).uniform(0.5, 1.5, cols).astype(np.float16)
    got = hip.recovered_row(ctox_hip.RecoveredRow(ctox_hip.TensorDType(dtype), w, cols,
                                                  ctox_hip.ScaleSlice.F16Le(s_in_f16.view(np.uint8)), 1.25))
    ref = orc.recovered_row(dtype, w.tobytes(), cols, ("f16le", s_in_f16.view(np.uint8)), 1.25)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    x = synth.activation("normal", cols, 9)[0]
    got = hip.recovered_row_matvec(ctox_hip.RecoveredRowMatVec(ctox_hip.TensorDType(dtype), w, x, 0.5))
    ref = orc.recovered_row_matvec(dtype, w.tobytes(), x, 0.5)
    assert abs(got - ref) <= 1e-4 * (abs(ref) + 1.0)


@pytest.mark.parametrize("dtype,rows,cols", [(1, 1000, 5120), (0, 333, 17408), (1, 17, 192)])
def test_registered_tiled_raw_launch(hip, orc, dtype, rows, cols):
    """Batch-1 raw launches on registered weights run the tiled kernel and
    agree with the oracle; after unregistering, the crate-layout kernels
    give the same rows to the stated tolerance."""
    torch = _torch()
    say(f"case registered tiled dtype={dtype} {rows}x{cols}")
    w = synth.random_matrix(dtype, rows, cols, 91)
    x = synth.activation("normal", cols, 92, 1)
    s_in = np.linspace(0.9, 1.1, cols).astype(np.float16)
    s_out = np.linspace(1.1, 0.9, rows).astype(np.float16)
    ref = orc.fused_matvec(dtype, w, rows, cols, x[0], ("f16le", s_in.view(np.uint8)), ("f16le", s_out.view(np.uint8)),
                           None, 0)
    dw = torch.from_numpy(w).cuda()
    dx = torch.from_numpy(x).cuda()
    dsi = torch.from_numpy(s_in.view(np.int16)).cuda()
    dso = torch.from_numpy(s_out.view(np.int16)).cuda()
    stream = torch.cuda.current_stream().cuda_stream
    hip.register_tiled_weights(ctox_hip.TensorDType(dtype), dw.data_ptr(), rows, cols, stream)
    outs = []
    for _ in range(2):
        dy = torch.full((1, rows), float("nan"), device="cuda")
        hip.launch_fused_matvec(ctox_hip.TensorDType(dtype), dw.data_ptr(), dx.data_ptr(), dsi.data_ptr(),
                                dso.data_ptr(), None, dy.data_ptr(), rows, cols, ctox_hip.Activation.Identity, 1, stream)
        torch.cuda.synchronize()
        outs.append(dy.cpu().numpy()[0])
    assert np.array_equal(outs[0], outs[1])
    check(outs[0], ref, "registered tiled")
    hip.unregister_tiled_weights(dw.data_ptr())
    dy = torch.empty((1, rows), device="cuda")
    hip.launch_fused_matvec(ctox_hip.TensorDType(dtype), dw.data_ptr(), dx.data_ptr(), dsi.data_ptr(), dso.data_ptr(),
                            None, dy.data_ptr(), rows, cols, ctox_hip.Activation.Identity, 1, stream)
    torch.cuda.synchronize()
    check(dy.cpu().numpy()[0], ref, "crate layout after unregister")


@pytest.mark.gpu
def test_artifact_mixed_recovered_upload(hip, orc, tmp_path):
    """A v2 `.ctoxq` mixed tensor with FP16 recovery scales, mapped and uploaded to HBM
    (models/qwen38_27b/src/loader.rs:362-402), equals the oracle on the same bytes."""
    from ctox_hip import artifact as A
    say("case artifact mixed recovered upload")
    torch = _torch()
    T = ctox_hip.TensorDType
    cols, r2, r4 = 1024, 48, 80
    q2 = synth.random_matrix(0, r2, cols, 11)
    q4 = synth.random_matrix(1, r4, cols, 12)
    rng = np.random.default_rng(13)
    s_in = (0.5 + rng.random(cols)).astype("<f2")
    s_out = (0.5 + rng.random(r2 + r4)).astype("<f2")
    segs = [ctox_hip.QuantSegment(0, 0, r2, T.Q2B64, 0, q2.size),
            ctox_hip.QuantSegment(1, r2, r2 + r4, T.Q4B64, q2.size, q4.size)]
    path = tmp_path / "mixed.ctoxq"
    A.ArtifactBuilder("test/qwen", "0123456789abcdef", "gfx950", 256, [
        A.PackedTensor("w", T.MixedQ2Q4B64, [r2 + r4, cols], np.concatenate([q2, q4]).tobytes(), segs),
        A.PackedTensor("w.s_in", T.F16, [cols], s_in.tobytes()),
        A.PackedTensor("w.s_out", T.F16, [r2 + r4], s_out.tobytes()),
    ]).write_new(path)
    art = A.ModelArtifact.open(path, A.ChecksumPolicy.AllTensors)
    m = A.upload_matrix(hip, art, "w")
    xs = synth.activation("normal", cols, 14, batch=2)
    dx = torch.from_numpy(np.ascontiguousarray(xs)).cuda()
    dy = torch.empty((xs.shape[0], r2 + r4), dtype=torch.float32, device="cuda")
    m.dispatch(dx.data_ptr(), xs.shape[0], dy.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = dy.cpu().numpy()
    m.close()
    raw = np.concatenate([q2, q4]).tobytes()
    for b in range(xs.shape[0]):
        ref = orc.fused_matvec(2, raw, r2 + r4, cols, xs[b], s_in=("f16le", s_in.view(np.uint8)),
                               s_out=("f16le", s_out.view(np.uint8)),
                               segments=[(0, 0, r2, 0, 0, q2.size), (1, r2, r2 + r4, 1, q2.size, q4.size)])
        check(got[b], ref, f"artifact mixed batch row {b}")


def test_calls_on_two_streams_are_ordered(hip, orc):
    """The backend's scratch (activation staging, combine slots) is shared:
    device calls issued back to back on two streams, with no host wait in
    between, still each see their own inputs (the second stream waits for
    the first)."""
    torch = _torch()
    say("case two streams")
    rows, cols = 5120, 17408
    op, parts = make_case(0, rows, cols, 31, "f16", bias=False, batch=1)
    m = hip.prepare(op)
    x2 = synth.activation("normal", cols, 32, 1)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    d1 = torch.from_numpy(parts[1]).cuda()
    d2 = torch.from_numpy(x2).cuda()
    y1 = torch.empty((1, rows), device="cuda")
    y2 = torch.empty((1, rows), device="cuda")
    torch.cuda.synchronize()
    for _ in range(3):
        m.dispatch(d1.data_ptr(), 1, y1.data_ptr(), s1.cuda_stream)
        m.dispatch(d2.data_ptr(), 1, y2.data_ptr(), s2.cuda_stream)
    torch.cuda.synchronize()
    w, x, osi, oso, b = parts
    check(y1.cpu().numpy()[0], orc.fused_matvec(0, w, rows, cols, x[0], osi, oso), "stream 1")
    check(y2.cpu().numpy()[0], orc.fused_matvec(0, w, rows, cols, x2[0], osi, oso), "stream 2")
    m.close()
