"""GPU parity of the layer glue kernels against the oracle.

* rms_norm (1 + w) and gated rms_norm: Q/src/reference.rs:38-93. The GPU
  reduces the sum of squares as a tree, the oracle sequentially, so outputs
  agree to 1e-5 relative (well inside the 1e-3 bar).
* swiglu / sigmoid_gate: Q/src/reference.rs:96-112 and :502-515, elementwise
  with the device expf (within a few ulp of glibc's).
* causal conv update: Q/src/reference.rs:159-187. The state shift is bit-exact;
  the dot runs in the oracle's order but contracted to fused multiply-adds,
  so outputs near zero (where the dot cancels) get an absolute 1e-6 floor.
* partial RoPE: Q/src/reference.rs:115-155, rows at consecutive positions.
  The angle is position * theta^(-2i/rd) in f32: one ulp of the device powf
  moves the angle by one ulp of its own magnitude, so the tolerance is
  4 ulp of the largest angle (times |x|), and exact outside the rotary dims.
"""
import sys

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).cuda()


@pytest.mark.parametrize("rows,cols", [(1, 5120), (5, 5120), (3, 128), (2, 17), (1, 1)])
def test_rms_norm(hip, orc, rows, cols):
    say(f"case rms_norm rows={rows} cols={cols}")
    rng = np.random.default_rng(cols + rows)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    w = (rng.standard_normal(cols) * 0.2).astype(np.float32)
    g = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    keep = [dev(x), dev(w), dev(g)]
    out = torch.empty(rows, cols, device="cuda")
    out2 = torch.empty(rows, cols, device="cuda")
    hip.rms_norm_device(keep[0].data_ptr(), rows, cols, keep[1].data_ptr(), 1e-6, out.data_ptr())
    hip.rms_norm_gated_device(keep[0].data_ptr(), keep[2].data_ptr(), rows, cols, keep[1].data_ptr(), 1e-6,
                              out2.data_ptr())
    torch.cuda.synchronize()
    ref = orc.rms_norm_1p_weight(x.reshape(-1), rows, cols, w, 1e-6).reshape(rows, cols)
    ref2 = orc.rms_norm_gated(x.reshape(-1), g.reshape(-1), rows, cols, w, 1e-6).reshape(rows, cols)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out2.cpu().numpy(), ref2, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("n", [1, 255, 17408, 100003])
def test_swiglu_sigmoid_gate(hip, orc, n):
    say(f"case swiglu/sigmoid n={n}")
    rng = np.random.default_rng(n)
    a = (rng.standard_normal(n) * 5).astype(np.float32)
    b = (rng.standard_normal(n) * 5).astype(np.float32)
    da, db = dev(a), dev(b)
    out = torch.empty(n, device="cuda")
    hip.swiglu_device(da.data_ptr(), db.data_ptr(), n, out.data_ptr())
    hip.sigmoid_gate_device(da.data_ptr(), db.data_ptr(), n)   # in place on a
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.cpu().numpy(), orc.swiglu(a, b), rtol=2e-6, atol=1e-30)
    ref = a.copy()
    orc.sigmoid_gate(ref, b)
    np.testing.assert_allclose(da.cpu().numpy(), ref, rtol=2e-6, atol=1e-30)


@pytest.mark.parametrize("channels,kernel", [(10240, 4), (300, 4), (7, 1), (33, 6)])
def test_causal_conv_update(hip, orc, channels, kernel):
    say(f"case conv channels={channels} kernel={kernel}")
    rng = np.random.default_rng(channels * kernel)
    state = rng.standard_normal((channels, kernel)).astype(np.float32)
    weight = rng.standard_normal((channels, kernel)).astype(np.float32)
    ds, dw = dev(state), dev(weight)
    ref_state = state.reshape(-1).copy()
    for step in range(3):  # consecutive decode steps carry the state
        x = rng.standard_normal(channels).astype(np.float32)
        dx = dev(x)
        out = torch.empty(channels, device="cuda")
        hip.causal_conv_update_device(dx.data_ptr(), ds.data_ptr(), dw.data_ptr(), channels, kernel, out.data_ptr())
        torch.cuda.synchronize()
        ref = orc.causal_conv_silu_update(x, ref_state, weight.reshape(-1), channels, kernel)
        assert np.array_equal(ds.cpu().numpy().reshape(-1), ref_state), step
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("rows,qh,kh,hd,rd,pos", [(1, 24, 4, 256, 64, 0), (5, 24, 4, 256, 64, 4093),
                                                   (2, 3, 1, 128, 128, 70000), (3, 2, 2, 10, 2, 12)])
def test_partial_rope(hip, orc, rows, qh, kh, hd, rd, pos):
    say(f"case rope rows={rows} qh={qh} kh={kh} hd={hd} rd={rd} pos={pos}")
    rng = np.random.default_rng(rows + hd + pos)
    q = rng.standard_normal((rows, qh, hd)).astype(np.float32)
    k = rng.standard_normal((rows, kh, hd)).astype(np.float32)
    dq, dk = dev(q), dev(k)
    hip.partial_rope_device(dq.data_ptr(), dk.data_ptr(), rows, qh, kh, hd, rd, pos, 1e7)
    torch.cuda.synchronize()
    gq, gk = dq.cpu().numpy(), dk.cpu().numpy()
    for t in range(rows):
        rq, rk = q[t].reshape(-1).copy(), k[t].reshape(-1).copy()
        orc.apply_partial_rope(rq, rk, qh, kh, hd, rd, pos + t, 1e7)
        tol = 4 * float(np.spacing(np.float32(max(pos + t, 1)))) * 2 * 4.5 + 1e-6
        for got, ref, src in ((gq[t], rq.reshape(qh, hd), q[t]), (gk[t], rk.reshape(kh, hd), k[t])):
            np.testing.assert_allclose(got[:, :rd], ref[:, :rd], rtol=0, atol=tol)
            assert np.array_equal(got[:, rd:], src[:, rd:])


def test_layer_ops_errors(hip):
    import ctox_hip
    t = torch.zeros(16, device="cuda")
    p = t.data_ptr()
    with pytest.raises(ctox_hip.ShapeError):
        hip.rms_norm_device(p, 1, 16, p, 0.0, p)
    with pytest.raises(ctox_hip.ShapeError):
        hip.rms_norm_device(p, 0, 16, p, 1e-6, p)
    with pytest.raises(ctox_hip.ShapeError):
        hip.swiglu_device(p, p, 0, p)
    with pytest.raises(ctox_hip.ShapeError):
        hip.partial_rope_device(p, p, 1, 1, 1, 8, 3, 0, 1e7)
    with pytest.raises(ctox_hip.ShapeError):
        hip.partial_rope_device(p, p, 1, 1, 1, 8, 10, 0, 1e7)
    with pytest.raises(ctox_hip.ShapeError):
        hip.causal_conv_update_device(p, p, p, 4, 0, p)


def test_strided_gates_and_conv_rows(hip, orc):
    """Gates and the causal conv over token rows of a fused projection
    output (stride > width), tokens applied in order."""
    say("case strided gates / conv rows")
    rng = np.random.default_rng(21)
    T, H, C, K, stride = 5, 48, 10240, 4, 16480
    rows = rng.standard_normal((T, stride)).astype(np.float32)
    a_log = rng.uniform(-2, 1, H).astype(np.float32)
    dt = rng.uniform(-1, 1, H).astype(np.float32)
    drows = dev(rows)
    ka, kd = dev(a_log), dev(dt)
    ld, be = torch.empty(T, H, device="cuda"), torch.empty(T, H, device="cuda")
    off_a, off_b = 16384, 16384 + H
    hip.gdn_gates_strided_device(drows.data_ptr() + off_a * 4, drows.data_ptr() + off_b * 4, stride, ka.data_ptr(),
                                 kd.data_ptr(), T, H, ld.data_ptr(), be.data_ptr())
    state = rng.standard_normal((C, K)).astype(np.float32)
    weight = rng.standard_normal((C, K)).astype(np.float32)
    ds, dw = dev(state), dev(weight)
    out = torch.empty(T, C, device="cuda")
    hip.causal_conv_rows_device(drows.data_ptr(), stride, ds.data_ptr(), dw.data_ptr(), C, K, T, out.data_ptr())
    torch.cuda.synchronize()
    ref_state = state.reshape(-1).copy()
    for t in range(T):
        rl, rb = orc.gdn_gates(rows[t, off_a:off_a + H], rows[t, off_b:off_b + H], a_log, dt)
        np.testing.assert_allclose(ld[t].cpu().numpy(), rl, rtol=4e-7, atol=1e-30)
        np.testing.assert_allclose(be[t].cpu().numpy(), rb, rtol=4e-7, atol=1e-30)
        ref = orc.causal_conv_silu_update(rows[t, :C], ref_state, weight.reshape(-1), C, K)
        np.testing.assert_allclose(out[t].cpu().numpy(), ref, rtol=2e-6, atol=1e-6)
    assert np.array_equal(ds.cpu().numpy().reshape(-1), ref_state)


@pytest.mark.parametrize("batch,with_delta,dtype,registered,rows,cols", [
    (1, True, 1, False, 300, 5120), (3, False, 1, False, 300, 5120), (5, True, 0, False, 300, 5120),
    (1, True, 1, True, 300, 5120), (1, False, 0, True, 300, 5120), (1, True, 0, True, 300, 5120),
    (1, True, 1, True, 1024, 256), (1, False, 1, True, 512, 256), (1, True, 0, True, 40, 1088)])
def test_norm_matvec(hip, orc, batch, with_delta, dtype, registered, rows, cols):
    """Residual add + (1 + w) RMS norm fused with the projection's activation
    staging (registered weights: inside the tiled matvec), against the oracle
    norm followed by the oracle fused matvec."""
    say(f"case norm_matvec batch={batch} delta={with_delta} dtype={dtype} registered={registered}")
    from ctox_hip import synth  # noqa: F401  (weights built here directly)
    rng = np.random.default_rng(batch * 10 + dtype)
    bb = 34 if dtype == 1 else 18
    blocks = rng.integers(0, 256, size=(rows, cols // 64, bb), dtype=np.uint8)
    scales = (np.abs(rng.standard_normal((rows, cols // 64))) * 0.02).astype(np.float16)
    blocks[:, :, :2] = scales.view(np.uint8).reshape(rows, cols // 64, 2)
    w_bytes = blocks.tobytes()
    s_in = rng.uniform(0.75, 1.25, cols).astype(np.float16)
    s_out = rng.uniform(0.75, 1.25, rows).astype(np.float16)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    d = rng.standard_normal((batch, cols)).astype(np.float32)
    nw = (rng.standard_normal(cols) * 0.1).astype(np.float32)
    dx, dd, dw = dev(x), dev(d), dev(nw)
    dwt = torch.from_numpy(np.frombuffer(w_bytes, np.uint8).copy()).cuda()
    dsi = torch.from_numpy(s_in.view(np.int16).copy()).cuda()
    dso = torch.from_numpy(s_out.view(np.int16).copy()).cuda()
    xo = torch.empty(batch, cols, device="cuda")
    no = torch.empty(batch, cols, device="cuda")
    out = torch.empty(batch, rows, device="cuda")
    hip_lib = __import__("ctox_hip").load_library()
    if registered:
        hip.register_tiled_weights(__import__("ctox_hip").TensorDType(dtype), dwt.data_ptr(), rows, cols)
    st = hip_lib.ctox_hip_norm_matvec_device(hip.handle, dx.data_ptr(), dd.data_ptr() if with_delta else None, 1, 0,
                                             xo.data_ptr() if with_delta else None, dw.data_ptr(), 1e-6,
                                             no.data_ptr(), dtype, dwt.data_ptr(), dsi.data_ptr(), dso.data_ptr(),
                                             out.data_ptr(), rows, cols, batch, None)
    assert st == 0, hip_lib.ctox_hip_last_error()
    torch.cuda.synchronize()
    for t in range(batch):
        h = (x[t] + d[t]) if with_delta else x[t]
        if with_delta:
            assert np.array_equal(xo[t].cpu().numpy(), h)
        y = orc.rms_norm_1p_weight(h, 1, cols, nw, 1e-6)
        np.testing.assert_allclose(no[t].cpu().numpy(), y, rtol=1e-5, atol=1e-6)
        ref = orc.fused_matvec(dtype, w_bytes, rows, cols, y, s_in=("f16le", s_in.view(np.uint8)),
                               s_out=("f16le", s_out.view(np.uint8)))
        np.testing.assert_allclose(out[t].cpu().numpy(), ref, rtol=1e-3, atol=1e-4 * float(np.abs(ref).max()))
    if registered:
        hip.unregister_tiled_weights(dwt.data_ptr())


class _Transform(ctypes.Structure):
    _fields_ = [("a", ctypes.c_void_p), ("b", ctypes.c_void_p), ("w", ctypes.c_void_p), ("mode", ctypes.c_uint32),
                ("a_stride", ctypes.c_uint32), ("b_stride", ctypes.c_uint32), ("off", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("eps", ctypes.c_float), ("res_h", ctypes.c_void_p),
                ("res_sums", ctypes.c_void_p), ("a_parts", ctypes.c_uint32), ("a_part_stride", ctypes.c_uint32)]


@pytest.mark.parametrize("mode,dtype,registered,hd,heads", [
    (1, 0, True, 128, 12), (2, 1, True, 128, 12), (3, 1, True, 128, 12), (1, 0, False, 128, 12),
    (2, 1, False, 128, 12), (3, 1, False, 128, 12), (2, 1, True, 64, 4), (3, 1, True, 256, 4), (1, 0, True, 64, 4)])
def test_transform_matvec(hip, orc, mode, dtype, registered, hd, heads):
    """Producer fused into a projection (swiglu -> down, gated norm ->
    out_proj, attention gate -> o_proj), batch 1, with the staging kernel or
    (registered weights) inside the tiled matvec, against the oracle producer
    followed by the oracle fused matvec."""
    import ctox_hip
    say(f"case transform_matvec mode={mode} dtype={dtype} registered={registered}")
    rng = np.random.default_rng(40 + mode)
    rows = 192
    cols = {1: 2048 if heads == 12 else 512, 2: heads * hd, 3: heads * hd}[mode]
    bb = 34 if dtype == 1 else 18
    blocks = rng.integers(0, 256, size=(rows, cols // 64, bb), dtype=np.uint8)
    blocks[:, :, :2] = (np.abs(rng.standard_normal((rows, cols // 64))) * 0.02).astype(np.float16).view(
        np.uint8).reshape(rows, cols // 64, 2)
    w_bytes = blocks.tobytes()
    s_in = rng.uniform(0.75, 1.25, cols).astype(np.float16)
    s_out = rng.uniform(0.75, 1.25, rows).astype(np.float16)
    nw = (rng.standard_normal(hd) * 0.1 + 1.0).astype(np.float32)
    if mode == 1:
        a = rng.standard_normal(2 * cols).astype(np.float32)
        b = None
        x = orc.swiglu(a[:cols], a[cols:])
        tr = _Transform(0, 0, 0, 1, 2 * cols, 0, cols, 0, 0.0)
    elif mode == 2:
        a = rng.standard_normal(cols).astype(np.float32)
        b = rng.standard_normal(cols).astype(np.float32)
        x = orc.rms_norm_gated(a, b, heads, hd, nw, 1e-6)
        tr = _Transform(0, 0, 0, 2, cols, cols, 0, hd, 1e-6)
    else:
        a = rng.standard_normal(cols).astype(np.float32)
        b = rng.standard_normal(2 * cols).astype(np.float32)
        x = a.copy()
        orc.sigmoid_gate(x, b.reshape(heads, 2 * hd)[:, hd:].reshape(-1))
        tr = _Transform(0, 0, 0, 3, cols, 2 * cols, 0, hd, 0.0)
    da, dw_norm = dev(a), dev(nw)
    db = dev(b) if b is not None else None
    tr.a = da.data_ptr()
    tr.b = db.data_ptr() if db is not None else None
    tr.w = dw_norm.data_ptr() if mode == 2 else None
    dwt = torch.from_numpy(np.frombuffer(w_bytes, np.uint8).copy()).cuda()
    dsi = torch.from_numpy(s_in.view(np.int16).copy()).cuda()
    dso = torch.from_numpy(s_out.view(np.int16).copy()).cuda()
    out = torch.full((1, rows), float("nan"), device="cuda")
    lib = ctox_hip.load_library()
    if registered:
        hip.register_tiled_weights(ctox_hip.TensorDType(dtype), dwt.data_ptr(), rows, cols)
    parts = ctypes.c_uint32(0)
    st = lib.ctox_hip_transform_matvec_device(hip.handle, ctypes.byref(tr), dtype, dwt.data_ptr(), dsi.data_ptr(),
                                              dso.data_ptr(), out.data_ptr(), rows, cols, 1, 0,
                                              ctypes.byref(parts), None)
    assert st == 0, lib.ctox_hip_last_error()
    torch.cuda.synchronize()
    if registered:
        hip.unregister_tiled_weights(dwt.data_ptr())
    ref = orc.fused_matvec(dtype, w_bytes, rows, cols, x, s_in=("f16le", s_in.view(np.uint8)),
                           s_out=("f16le", s_out.view(np.uint8)))
    got = out[0].cpu().numpy()
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    assert np.all(np.abs(got - ref) <= 1e-3 * (np.abs(ref) + rms)), float(np.abs(got - ref).max())


@pytest.mark.parametrize("rows,cols", [(5120, 2048), (320, 512)])
def test_residual_sums_chain(hip, orc, rows, cols):
    """A projection producing a residual delta (swiglu -> down, registered
    weights, batch 1) also writes per-16-row sums of (h + delta)^2, checked
    against float64; the next norm-matvec given those sums matches the one
    that reduces the row itself (both against the oracle norm + matvec)."""
    import ctox_hip
    say(f"case residual sums rows={rows} cols={cols}")
    rng = np.random.default_rng(rows + cols)
    lib = ctox_hip.load_library()

    def qmat(r, c, dtype):
        bb = 34 if dtype == 1 else 18
        blocks = rng.integers(0, 256, size=(r, c // 64, bb), dtype=np.uint8)
        blocks[:, :, :2] = (np.abs(rng.standard_normal((r, c // 64))) * 0.02).astype(np.float16).view(
            np.uint8).reshape(r, c // 64, 2)
        return blocks.tobytes()

    w1 = qmat(rows, cols, 0)                      # producer: down-like, out [rows]
    w2 = qmat(256, rows, 1)                       # consumer: reads the rows-wide residual
    a = rng.standard_normal(2 * cols).astype(np.float32)
    hres = rng.standard_normal(rows).astype(np.float32)
    nw = (rng.standard_normal(rows) * 0.1).astype(np.float32)
    d1 = torch.from_numpy(np.frombuffer(w1, np.uint8).copy()).cuda()
    d2 = torch.from_numpy(np.frombuffer(w2, np.uint8).copy()).cuda()
    hip.register_tiled_weights(ctox_hip.TensorDType(0), d1.data_ptr(), rows, cols)
    hip.register_tiled_weights(ctox_hip.TensorDType(1), d2.data_ptr(), 256, rows)
    da, dh, dw = dev(a), dev(hres), dev(nw)
    delta = torch.empty(rows, device="cuda")
    tiles = (rows + 15) // 16
    sums = torch.full((tiles,), float("nan"), device="cuda")
    tr = _Transform(da.data_ptr(), None, None, 1, 2 * cols, 0, cols, 0, 0.0, dh.data_ptr(), sums.data_ptr())
    parts = ctypes.c_uint32(0)
    st = lib.ctox_hip_transform_matvec_device(hip.handle, ctypes.byref(tr), 0, d1.data_ptr(), None, None,
                                              delta.data_ptr(), rows, cols, 1, 1, ctypes.byref(parts), None)
    assert st == 0, lib.ctox_hip_last_error()
    torch.cuda.synchronize()
    h = (hres + delta.cpu().numpy()).astype(np.float32)
    want = np.array([np.sum(h[t * 16:(t + 1) * 16].astype(np.float64) ** 2) for t in range(tiles)])
    np.testing.assert_allclose(sums.cpu().numpy(), want, rtol=1e-5)
    outs = []
    for use in (False, True):
        xo = torch.empty(rows, device="cuda")
        out = torch.empty(256, device="cuda")
        st = lib.ctox_hip_norm_matvec_sums_device(hip.handle, dh.data_ptr(), delta.data_ptr(), 1, 0, xo.data_ptr(),
                                                  dw.data_ptr(), 1e-6, None, 1, d2.data_ptr(), None, None,
                                                  out.data_ptr(), 256, rows, 1,
                                                  sums.data_ptr() if use else None, tiles if use else 0, None)
        assert st == 0, lib.ctox_hip_last_error()
        torch.cuda.synchronize()
        assert np.array_equal(xo.cpu().numpy(), h)
        outs.append(out.cpu().numpy())
    y = orc.rms_norm_1p_weight(h, 1, rows, nw, 1e-6)
    ref = orc.fused_matvec(1, w2, 256, rows, y)
    for got in outs:
        np.testing.assert_allclose(got, ref, rtol=1e-3, atol=1e-4 * float(np.abs(ref).max()))
    np.testing.assert_allclose(outs[1], outs[0], rtol=1e-5, atol=1e-6 * float(np.abs(ref).max()))
    # Unregistered weights cannot produce the sums: fails closed.
    hip.unregister_tiled_weights(d1.data_ptr())
    st = lib.ctox_hip_transform_matvec_device(hip.handle, ctypes.byref(tr), 0, d1.data_ptr(), None, None,
                                              delta.data_ptr(), rows, cols, 1, 1, ctypes.byref(parts), None)
    assert st == 5, st  # CTOX_ERR_UNSUPPORTED_OPERATION
    hip.unregister_tiled_weights(d2.data_ptr())


@pytest.mark.parametrize("batch", [1, 5])
@pytest.mark.parametrize("cols", [5120, 1024])
def test_gate_up_partials_chain(hip, orc, cols, batch):
    """gate|up as a norm-matvec that leaves its chunk partials
    (ctox_hip_norm_matvec_parts_device on registered weights: built in the
    kernel at batch 1, on staged rows at batch 5), then swiglu -> down
    adding them (in its in-kernel build at batch 1, in its staging at
    batch 5; a_parts), against the oracle norm, gate|up, swiglu and down per
    row; the partials' sum equals the finished gate|up rows within
    rounding."""
    import ctox_hip
    say(f"case gate|up partials cols={cols} batch={batch}")
    rng = np.random.default_rng(cols + batch)
    lib = ctox_hip.load_library()
    inter, out_rows = 1024, 256

    def qmat(r, c, dtype):
        bb = 34 if dtype == 1 else 18
        blocks = rng.integers(0, 256, size=(r, c // 64, bb), dtype=np.uint8)
        blocks[:, :, :2] = (np.abs(rng.standard_normal((r, c // 64))) * 0.02).astype(np.float16).view(
            np.uint8).reshape(r, c // 64, 2)
        return blocks.tobytes()

    wgu, wdn = qmat(2 * inter, cols, 1), qmat(out_rows, inter, 0)
    so = rng.uniform(0.75, 1.25, 2 * inter).astype(np.float16)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    nw = (rng.standard_normal(cols) * 0.1).astype(np.float32)
    dgu = torch.from_numpy(np.frombuffer(wgu, np.uint8).copy()).cuda()
    ddn = torch.from_numpy(np.frombuffer(wdn, np.uint8).copy()).cuda()
    dso = torch.from_numpy(so.view(np.int16).copy()).cuda()
    hip.register_tiled_weights(ctox_hip.TensorDType(1), dgu.data_ptr(), 2 * inter, cols)
    hip.register_tiled_weights(ctox_hip.TensorDType(0), ddn.data_ptr(), out_rows, inter)
    dx, dw = dev(x), dev(nw)
    gu = torch.full((6, batch, 2 * inter), float("nan"), device="cuda")
    parts = ctypes.c_uint32(0)
    st = lib.ctox_hip_norm_matvec_parts_device(hip.handle, dx.data_ptr(), None, 1, 0, None, dw.data_ptr(), 1e-6, None,
                                               1, dgu.data_ptr(), None, dso.data_ptr(), gu.data_ptr(), 2 * inter,
                                               cols, batch, None, 0, 6, ctypes.byref(parts), None)
    assert st == 0, lib.ctox_hip_last_error()
    n = parts.value
    assert n == (cols // 64 + 15) // 16 or n == 1
    assert n > 1 or cols == 1024
    out = torch.empty(batch, out_rows, device="cuda")
    tr = _Transform(gu.data_ptr(), None, None, 1, 2 * inter, 0, inter, 0, 0.0, None, None, n, batch * 2 * inter)
    pp = ctypes.c_uint32(0)
    st = lib.ctox_hip_transform_matvec_device(hip.handle, ctypes.byref(tr), 0, ddn.data_ptr(), None, None,
                                              out.data_ptr(), out_rows, inter, batch, 1, ctypes.byref(pp), None)
    assert st == 0, lib.ctox_hip_last_error()
    torch.cuda.synchronize()
    for t in range(batch):
        y = orc.rms_norm_1p_weight(x[t], 1, cols, nw, 1e-6)
        ref_gu = orc.fused_matvec(1, wgu, 2 * inter, cols, y, s_out=("f16le", so.view(np.uint8)))
        got_gu = gu[:n, t].cpu().numpy().sum(axis=0)
        np.testing.assert_allclose(got_gu, ref_gu, rtol=1e-3, atol=1e-4 * float(np.abs(ref_gu).max()))
        ref = orc.fused_matvec(0, wdn, out_rows, inter, orc.swiglu(ref_gu[:inter], ref_gu[inter:]))
        np.testing.assert_allclose(out[t].cpu().numpy(), ref, rtol=1e-3, atol=1e-4 * float(np.abs(ref).max()))
    hip.unregister_tiled_weights(dgu.data_ptr())
    hip.unregister_tiled_weights(ddn.data_ptr())


def _qmat(rng, r, c, dtype):
    bb = 34 if dtype == 1 else 18
    blocks = rng.integers(0, 256, size=(r, c // 64, bb), dtype=np.uint8)
    blocks[:, :, :2] = (np.abs(rng.standard_normal((r, c // 64))) * 0.02).astype(np.float16).view(
        np.uint8).reshape(r, c // 64, 2)
    return blocks.tobytes()


def _close_rows(got, ref):
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    assert np.all(np.abs(got - ref) <= 1e-3 * (np.abs(ref) + rms)), float(np.abs(got - ref).max())


@pytest.mark.parametrize("batch", [2, 3, 5])
@pytest.mark.parametrize("mode,dtype,hd,heads,rows", [(1, 0, 0, 0, 200), (2, 1, 128, 12, 200), (3, 1, 256, 6, 200),
                                                      (2, 0, 64, 8, 200), (1, 0, 0, 0, 8256)])
def test_transform_matvec_rows_built_in_kernel(hip, orc, batch, mode, dtype, hd, heads, rows):
    """2..5 rows of a producer fused into a projection on registered weights
    (up to 8 Mi weights ctox_q*_mv_tilemx*, every row's fragments built in
    the launch; the 8256 x 5120 case runs the staging launch and the staged
    kernel), with the residual sums of every row, against the oracle producer
    + matvec per row and float64 sums. Widths with a partial last
    1024-column chunk and ragged row tiles."""
    import ctox_hip
    say(f"case transform rows batch={batch} mode={mode} dtype={dtype} rows={rows}")
    rng = np.random.default_rng(100 * batch + 10 * mode + dtype)
    cols = {1: 1536 if rows < 1000 else 5120, 2: heads * hd, 3: heads * hd}[mode]
    w = _qmat(rng, rows, cols, dtype)
    s_in = rng.uniform(0.75, 1.25, cols).astype(np.float16)
    s_out = rng.uniform(0.75, 1.25, rows).astype(np.float16)
    nw = (rng.standard_normal(max(hd, 1)) * 0.1 + 1.0).astype(np.float32)
    astr = {1: 2 * cols + 64, 2: cols + 64, 3: cols + 32}[mode]
    bstr = {1: 0, 2: cols + 128, 3: 2 * cols + 64}[mode]
    a = rng.standard_normal((batch, astr)).astype(np.float32)
    b = rng.standard_normal((batch, max(bstr, 1))).astype(np.float32)
    xs = []
    for t in range(batch):
        if mode == 1:
            xs.append(orc.swiglu(a[t, :cols], a[t, cols:2 * cols]))
        elif mode == 2:
            xs.append(orc.rms_norm_gated(a[t, :cols], b[t, :cols], heads, hd, nw, 1e-6))
        else:
            x = a[t, :cols].copy()
            orc.sigmoid_gate(x, b[t, :2 * cols].reshape(heads, 2 * hd)[:, hd:].reshape(-1))
            xs.append(x)
    hres = rng.standard_normal((batch, rows)).astype(np.float32)
    da, db, dwn, dh = dev(a), dev(b), dev(nw), dev(hres)
    tiles = (rows + 15) // 16
    sums = torch.full((batch, tiles), float("nan"), device="cuda")
    tr = _Transform(da.data_ptr(), db.data_ptr() if mode != 1 else None, dwn.data_ptr() if mode == 2 else None, mode,
                    astr, bstr, cols if mode == 1 else 0, hd, 1e-6, dh.data_ptr(), sums.data_ptr())
    dwt = torch.from_numpy(np.frombuffer(w, np.uint8).copy()).cuda()
    dsi = torch.from_numpy(s_in.view(np.int16).copy()).cuda()
    dso = torch.from_numpy(s_out.view(np.int16).copy()).cuda()
    out = torch.full((batch, rows), float("nan"), device="cuda")
    lib = ctox_hip.load_library()
    hip.register_tiled_weights(ctox_hip.TensorDType(dtype), dwt.data_ptr(), rows, cols)
    try:
        parts = ctypes.c_uint32(0)
        st = lib.ctox_hip_transform_matvec_device(hip.handle, ctypes.byref(tr), dtype, dwt.data_ptr(), dsi.data_ptr(),
                                                  dso.data_ptr(), out.data_ptr(), rows, cols, batch, 1,
                                                  ctypes.byref(parts), None)
        assert st == 0, lib.ctox_hip_last_error()
        torch.cuda.synchronize()
    finally:
        hip.unregister_tiled_weights(dwt.data_ptr())
    got = out.cpu().numpy()
    for t in range(batch):
        ref = orc.fused_matvec(dtype, w, rows, cols, xs[t], s_in=("f16le", s_in.view(np.uint8)),
                               s_out=("f16le", s_out.view(np.uint8)))
        _close_rows(got[t], ref)
        h = (hres[t] + got[t]).astype(np.float64)
        want = np.array([np.sum(h[i * 16:(i + 1) * 16] ** 2) for i in range(tiles)])
        np.testing.assert_allclose(sums[t].cpu().numpy(), want, rtol=1e-5)


@pytest.mark.parametrize("batch", [2, 4, 5, 8])
@pytest.mark.parametrize("with_delta", [True, False])
@pytest.mark.parametrize("dtype,rows,cols", [(1, 300, 5120), (0, 64, 1536), (1, 2048, 5120)])
def test_norm_matvec_rows_with_sums(hip, orc, batch, with_delta, dtype, rows, cols):
    """Residual add + (1 + w) RMS norm + projection of 2..8 rows from the
    producer's per-tile sums (2..5 rows of a small matrix: ctox_q*_mv_tilemx*,
    built in the launch; 8 rows or more than 8 Mi weights: the staging
    launch reads the sums), against the oracle norm and matvec per row; the
    residual and normalized rows are written once."""
    import ctox_hip
    say(f"case norm rows batch={batch} delta={with_delta} dtype={dtype} {rows}x{cols}")
    rng = np.random.default_rng(batch * 7 + dtype + with_delta)
    w = _qmat(rng, rows, cols, dtype)
    s_in = rng.uniform(0.75, 1.25, cols).astype(np.float16)
    s_out = rng.uniform(0.75, 1.25, rows).astype(np.float16)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    d = rng.standard_normal((batch, cols)).astype(np.float32)
    nw = (rng.standard_normal(cols) * 0.1).astype(np.float32)
    h = (x + d) if with_delta else x
    tiles = (cols + 15) // 16
    sums = np.array([[np.sum(h[t, i * 16:(i + 1) * 16].astype(np.float64) ** 2) for i in range(tiles)]
                     for t in range(batch)], np.float32)
    dx, dd, dw, ds = dev(x), dev(d), dev(nw), dev(sums)
    dwt = torch.from_numpy(np.frombuffer(w, np.uint8).copy()).cuda()
    dsi = torch.from_numpy(s_in.view(np.int16).copy()).cuda()
    dso = torch.from_numpy(s_out.view(np.int16).copy()).cuda()
    xo = torch.full((batch, cols), float("nan"), device="cuda")
    no = torch.full((batch, cols), float("nan"), device="cuda")
    out = torch.full((batch, rows), float("nan"), device="cuda")
    lib = ctox_hip.load_library()
    hip.register_tiled_weights(ctox_hip.TensorDType(dtype), dwt.data_ptr(), rows, cols)
    try:
        st = lib.ctox_hip_norm_matvec_sums_device(hip.handle, dx.data_ptr(), dd.data_ptr() if with_delta else None, 1,
                                                  0, xo.data_ptr() if with_delta else None, dw.data_ptr(), 1e-6,
                                                  no.data_ptr(), dtype, dwt.data_ptr(), dsi.data_ptr(), dso.data_ptr(),
                                                  out.data_ptr(), rows, cols, batch, ds.data_ptr(), tiles, None)
        assert st == 0, lib.ctox_hip_last_error()
        torch.cuda.synchronize()
    finally:
        hip.unregister_tiled_weights(dwt.data_ptr())
    for t in range(batch):
        if with_delta:
            assert np.array_equal(xo[t].cpu().numpy(), h[t])
        y = orc.rms_norm_1p_weight(h[t], 1, cols, nw, 1e-6)
        np.testing.assert_allclose(no[t].cpu().numpy(), y, rtol=1e-5, atol=1e-6)
        ref = orc.fused_matvec(dtype, w, rows, cols, y, s_in=("f16le", s_in.view(np.uint8)),
                               s_out=("f16le", s_out.view(np.uint8)))
        _close_rows(out[t].cpu().numpy(), ref)


@pytest.mark.parametrize("batch", [2, 3, 5])
@pytest.mark.parametrize("dtype", [0, 1])
def test_raw_launch_rows_built_in_kernel(hip, orc, batch, dtype):
    """The raw 9-parameter launch on registered weights with 2..5 rows (no
    staging launch) against the oracle per row, with bias and SiLU."""
    import ctox_hip
    say(f"case raw rows batch={batch} dtype={dtype}")
    rng = np.random.default_rng(batch + 5 * dtype)
    rows, cols = 333, 3072
    w = _qmat(rng, rows, cols, dtype)
    s_in = rng.uniform(0.75, 1.25, cols).astype(np.float16)
    s_out = rng.uniform(0.75, 1.25, rows).astype(np.float16)
    bias = (rng.standard_normal(rows) * 0.05).astype(np.float32)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    dwt = torch.from_numpy(np.frombuffer(w, np.uint8).copy()).cuda()
    dsi = torch.from_numpy(s_in.view(np.int16).copy()).cuda()
    dso = torch.from_numpy(s_out.view(np.int16).copy()).cuda()
    dx, db = dev(x), dev(bias)
    out = torch.full((batch, rows), float("nan"), device="cuda")
    hip.register_tiled_weights(ctox_hip.TensorDType(dtype), dwt.data_ptr(), rows, cols)
    try:
        hip.launch_fused_matvec(ctox_hip.TensorDType(dtype), dwt.data_ptr(), dx.data_ptr(), dsi.data_ptr(),
                                dso.data_ptr(), db.data_ptr(), out.data_ptr(), rows, cols, ctox_hip.Activation.Silu,
                                batch, None)
        torch.cuda.synchronize()
    finally:
        hip.unregister_tiled_weights(dwt.data_ptr())
    for t in range(batch):
        ref = orc.fused_matvec(dtype, w, rows, cols, x[t], s_in=("f16le", s_in.view(np.uint8)),
                               s_out=("f16le", s_out.view(np.uint8)), bias=bias, activation=1)
        _close_rows(out[t].cpu().numpy(), ref)
