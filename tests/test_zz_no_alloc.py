"""The allocation-free raw launch (ctox_hip_launch_fused_matvec_noalloc:
combine slots in a static device array) against the allocating raw launch
(ctox_hip_launch_fused_matvec) on the same registered weights, on calls in a
row, each smaller than the one before, for 1 and 3 rows, and with both ways
the chunks meet forced (CTOX_ARRIVE=0: the last chunk combines; =1: the last
to arrive combines, using the arrival counts in the static array's last
256 KiB, which must be back at zero for the next call):

* identical outputs where both launches build the activation fragments the
  same way (every Q2 case, small Q4 matrices);
* a large Q4 matrix at 3 rows, where the allocating launch stages 21-bit
  fragments and the allocation-free one builds 22-bit fragments in the
  kernel: both within the oracle tolerance and within 2^-20 relative of
  each other.

Every output is also checked against the oracle. A matrix whose combine
slots do not fit the static array is refused with CTOX_ERR_MEMORY_BUDGET."""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _case(rng, dtype, rows, cols, batch):
    bb = 34 if dtype == 1 else 18
    blocks = rng.integers(0, 256, size=(rows, cols // 64, bb), dtype=np.uint8)
    blocks[:, :, :2] = (np.abs(rng.standard_normal((rows, cols // 64))) * 0.02).astype(np.float16).view(
        np.uint8).reshape(rows, cols // 64, 2)
    w = blocks.tobytes()
    s_in = rng.uniform(0.75, 1.25, cols).astype(np.float16)
    s_out = rng.uniform(0.75, 1.25, rows).astype(np.float16)
    bias = (rng.standard_normal(rows) * 0.05).astype(np.float32)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    return w, s_in, s_out, bias, x


@pytest.mark.parametrize("arrive", [None, "0", "1"])
@pytest.mark.parametrize("batch", [1, 3])
def test_noalloc_launch_equals_allocating_launch(hip, orc, batch, arrive, monkeypatch):
    import torch
    import ctox_hip
    lib = ctox_hip.load_library()
    if arrive is not None:  # a backend of this test's own reads CTOX_ARRIVE at creation
        monkeypatch.setenv("CTOX_ARRIVE", arrive)
        hip = ctox_hip.HipBackend(0)
    try:
        _run_cases(hip, orc, lib, batch, arrive)
    finally:
        if arrive is not None:
            hip.close()


def _run_cases(hip, orc, lib, batch, arrive):
    import torch
    import ctox_hip
    rng = np.random.default_rng(batch)
    stream = torch.cuda.current_stream().cuda_stream
    # large matrices (17 and 5 column chunks), then a smaller one
    cases = [(0, 5120, 17408, True), (1, 17408, 5120, batch == 1), (1, 700, 2112, True)]
    for dtype, rows, cols, exact in cases:
        say(f"case noalloc arrive={arrive} batch={batch} dtype={dtype} {rows}x{cols}")
        w, s_in, s_out, bias, x = _case(rng, dtype, rows, cols, batch)
        dw = torch.from_numpy(np.frombuffer(w, np.uint8).copy()).cuda()
        dx = torch.from_numpy(x).cuda()
        dsi = torch.from_numpy(s_in.view(np.int16).copy()).cuda()
        dso = torch.from_numpy(s_out.view(np.int16).copy()).cuda()
        db = torch.from_numpy(bias).cuda()
        hip.register_tiled_weights(ctox_hip.TensorDType(dtype), dw.data_ptr(), rows, cols)
        try:
            outs = []
            for fn in (lib.ctox_hip_launch_fused_matvec, lib.ctox_hip_launch_fused_matvec_noalloc):
                y = torch.full((batch, rows), float("nan"), device="cuda")
                st = fn(hip.handle, dtype, dw.data_ptr(), dx.data_ptr(), dsi.data_ptr(), dso.data_ptr(), db.data_ptr(),
                        y.data_ptr(), rows, cols, 1, batch, stream)
                assert st == 0, lib.ctox_hip_last_error()
                torch.cuda.synchronize()
                outs.append(y.cpu().numpy())
            if exact:
                assert np.array_equal(outs[0], outs[1])
            else:
                scale = float(np.max(np.abs(outs[0])))
                assert np.max(np.abs(outs[0] - outs[1])) <= 2.0 ** -20 * scale
            for r in range(batch):
                ref = orc.fused_matvec(dtype, w, rows, cols, x[r], s_in=("f16le", s_in.view(np.uint8)),
                                       s_out=("f16le", s_out.view(np.uint8)), bias=bias, activation=1)
                rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
                for o in outs:
                    assert np.all(np.abs(o[r] - ref) <= 1e-3 * (np.abs(ref) + rms))
        finally:
            hip.unregister_tiled_weights(dw.data_ptr())


def test_noalloc_refuses_what_does_not_fit(hip):
    import torch
    import ctox_hip
    lib = ctox_hip.load_library()
    # LM-head shape at 5 rows: (5 - 1) chunks x 5 rows x 151936 rows x 8 B > 8 MiB
    rows, cols, batch = 151936, 5120, 5
    say("case noalloc refuses an oversized combine")
    dw = torch.zeros(rows * cols // 64 * 34, dtype=torch.uint8, device="cuda")
    dx = torch.zeros(batch, cols, device="cuda")
    y = torch.zeros(batch, rows, device="cuda")
    hip.register_tiled_weights(ctox_hip.TensorDType(1), dw.data_ptr(), rows, cols)
    try:
        st = lib.ctox_hip_launch_fused_matvec_noalloc(hip.handle, 1, dw.data_ptr(), dx.data_ptr(), None, None, None,
                                                      y.data_ptr(), rows, cols, 0, batch, None)
        assert st == 6, st  # CTOX_ERR_MEMORY_BUDGET
        # unregistered weights are refused too
        st = lib.ctox_hip_launch_fused_matvec_noalloc(hip.handle, 1, dx.data_ptr(), dx.data_ptr(), None, None, None,
                                                      y.data_ptr(), 16, 64, 0, 1, None)
        assert st == 5, st  # CTOX_ERR_UNSUPPORTED_OPERATION
    finally:
        hip.unregister_tiled_weights(dw.data_ptr())
