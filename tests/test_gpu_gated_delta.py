"""GPU parity of the fp32 gated-delta recurrence against the C oracle
(Q/src/reference.rs:230-415).

Tolerances: outputs elementwise within
1e-3 * (|ref| + rms(ref)); state within 1e-4 * (|ref| + rms(ref)). The
crate's golden vectors (2e-6) are checked at their own tolerance.
"""
import json
import math
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "crate_goldens.json")))


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def close(got, ref, rtol, what):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    rms = math.sqrt(float(np.mean(ref ** 2)))
    d = np.abs(got - ref)
    assert np.all(d <= rtol * (np.abs(ref) + rms)), f"{what}: max {d.max()} rms {rms}"


def gdn_inputs(tokens, heads, key_heads, dk, dv, seed):
    """q, k L2-normalised N(0,1) over key_heads, repeated to heads; v N(0,1);
    decay gate exp(-softplus(N)) (log_decay = -softplus(N)); beta = sigmoid(N)."""
    rng = np.random.default_rng(seed)
    rep = heads // key_heads
    qk = rng.standard_normal((2, tokens, key_heads, dk)).astype(np.float32)
    qk /= np.linalg.norm(qk, axis=-1, keepdims=True)
    q = np.repeat(qk[0], rep, axis=1).reshape(tokens, -1)
    k = np.repeat(qk[1], rep, axis=1).reshape(tokens, -1)
    v = rng.standard_normal((tokens, heads * dv)).astype(np.float32)
    n = rng.standard_normal((tokens, heads)).astype(np.float32)
    log_decay = (-np.logaddexp(0.0, n)).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((tokens, heads))))).astype(np.float32)
    return q, k, v, log_decay, beta


def test_golden_step_and_sequence(hip):
    say("case gdn goldens")
    g = GOLD["delta_step"]
    st = np.array(g["state"], np.float32)
    out = hip.gated_delta_step(g["q"], g["k"], g["v"], g["log_decay"], g["beta"], st, g["heads"], g["key_dim"],
                               g["value_dim"])
    assert np.max(np.abs(out - g["out"])) <= g["tol"] and np.max(np.abs(st - g["state_out"])) <= g["tol"]
    g = GOLD["delta_sequence"]
    st = np.array(g["state"], np.float32)
    out = hip.gated_delta_sequence(g["q"], g["k"], g["v"], g["log_decay"], g["beta"], st, g["tokens"], g["heads"],
                                   g["key_dim"], g["value_dim"])
    assert np.max(np.abs(out - g["out"])) <= g["tol"] and np.max(np.abs(st - g["state_out"])) <= g["tol"]


@pytest.mark.parametrize("heads,key_heads", [(32, 16), (48, 16)])
def test_decode_step_vs_oracle(hip, orc, heads, key_heads):
    say(f"case gdn decode heads={heads}")
    dk = dv = 128
    q, k, v, ld, be = gdn_inputs(17, heads, key_heads, dk, dv, heads)
    st_ref = np.zeros(heads * dk * dv, np.float32)
    # warm the state with 16 tokens (oracle), then one decode step on both
    orc.gated_delta_sequence(q[:16], k[:16], v[:16], ld[:16], be[:16], st_ref, 16, heads, dk, dv)
    st_gpu = st_ref.copy()
    ref = orc.gated_delta_step(q[16], k[16], v[16], ld[16], be[16], st_ref, heads, dk, dv)
    got = hip.gated_delta_step(q[16], k[16], v[16], ld[16], be[16], st_gpu, heads, dk, dv)
    close(got, ref, 1e-3, "output")
    close(st_gpu, st_ref, 1e-4, "state")


@pytest.mark.parametrize("chunk", [0, 64])
def test_sequence_vs_oracle(hip, orc, chunk):
    say(f"case gdn sequence chunk={chunk}")
    heads, dk, dv, T = 32, 128, 128, 512
    q, k, v, ld, be = gdn_inputs(T, heads, 16, dk, dv, 5)
    st_ref = (np.random.default_rng(6).standard_normal(heads * dk * dv) * 0.1).astype(np.float32)
    st_gpu = st_ref.copy()
    ref = orc.gated_delta_sequence(q, k, v, ld, be, st_ref, T, heads, dk, dv)
    got = hip.gated_delta_sequence(q, k, v, ld, be, st_gpu, T, heads, dk, dv, chunk)
    close(got, ref, 1e-3, "output")
    close(st_gpu, st_ref, 1e-4, "state")


@pytest.mark.parametrize("case", [(150, 2, 96, 40, 64), (150, 3, 128, 128, 16), (70, 1, 5, 7, 1),
                                  (64, 4, 128, 128, 64), (65, 2, 128, 128, 64), (33, 2, 64, 128, 7)])
def test_chunked_prefill_ragged(hip, orc, case):
    """Chunked (WY) path: partial last chunks, chunk lengths 1..64, dims below 128."""
    T, heads, dk, dv, chunk = case
    say(f"case gdn chunked {case}")
    q, k, v, ld, be = gdn_inputs(T, heads, heads, dk, dv, T + dk)
    st_ref = (np.random.default_rng(T).standard_normal(heads * dk * dv) * 0.1).astype(np.float32)
    st_gpu = st_ref.copy()
    ref = orc.gated_delta_sequence(q, k, v, ld, be, st_ref, T, heads, dk, dv)
    got = hip.gated_delta_sequence(q, k, v, ld, be, st_gpu, T, heads, dk, dv, chunk)
    close(got, ref, 1e-3, "output")
    close(st_gpu, st_ref, 1e-4, "state")


@pytest.mark.parametrize("T", [1024, 4096])
def test_chunked_prefill_long(hip, orc, T):
    """BASELINE config 4 shapes through the chunk-64 path, up to the config's
    full 4096-token prefill."""
    say(f"case gdn chunked long T={T}")
    heads, dk, dv = 32, 128, 128
    q, k, v, ld, be = gdn_inputs(T, heads, 16, dk, dv, 11)
    st_ref = np.zeros(heads * dk * dv, np.float32)
    st_gpu = st_ref.copy()
    ref = orc.gated_delta_sequence(q, k, v, ld, be, st_ref, T, heads, dk, dv)
    got = hip.gated_delta_sequence(q, k, v, ld, be, st_gpu, T, heads, dk, dv, 64)
    close(got, ref, 1e-3, "output")
    close(st_gpu, st_ref, 1e-4, "state")


@pytest.mark.parametrize("dims", [(3, 5, 7), (2, 64, 96), (4, 256, 128), (1, 1, 1)])
def test_ragged_dims(hip, orc, dims):
    heads, dk, dv = dims
    say(f"case gdn ragged {dims}")
    rng = np.random.default_rng(sum(dims))
    T = 9
    q = rng.standard_normal((T, heads * dk)).astype(np.float32)
    k = rng.standard_normal((T, heads * dk)).astype(np.float32)
    v = rng.standard_normal((T, heads * dv)).astype(np.float32)
    ld = -rng.uniform(0.01, 1.0, (T, heads)).astype(np.float32)
    be = rng.uniform(0.0, 1.0, (T, heads)).astype(np.float32)
    st_ref = rng.standard_normal(heads * dk * dv).astype(np.float32)
    st_gpu = st_ref.copy()
    ref = orc.gated_delta_sequence(q, k, v, ld, be, st_ref, T, heads, dk, dv)
    got = hip.gated_delta_sequence(q, k, v, ld, be, st_gpu, T, heads, dk, dv, 0)
    close(got, ref, 1e-3, "output")
    close(st_gpu, st_ref, 1e-4, "state")


def test_errors(hip):
    import ctox_hip
    st = np.zeros(2 * 3 * 2, np.float32)
    with pytest.raises(ctox_hip.InvalidArtifact):
        hip.gated_delta_step([np.nan] * 6, [1.0] * 6, [1.0] * 4, [0.0, 0.0], [0.5, 0.5], st, 2, 3, 2)
    st[0] = np.inf
    with pytest.raises(ctox_hip.ShapeError):
        hip.gated_delta_step([1.0] * 6, [1.0] * 6, [1.0] * 4, [0.0, 0.0], [0.5, 0.5], st, 2, 3, 2)
    with pytest.raises(ctox_hip.UnsupportedOperation):
        hip.gated_delta_step([1.0] * 300, [1.0] * 300, [1.0], [0.0], [0.5], np.zeros(300, np.float32), 1, 300, 1)


@pytest.mark.parametrize("tokens,chunk", [(1, 0), (5, 0), (40, 16)])
def test_strided_repeated_key_heads(hip, orc, tokens, chunk):
    """q, k, v read in place from a fused [q | k | v] token row with 16 key
    heads repeated to 48 value heads (Q/src/decoder.rs:868-913) against the
    oracle on explicitly repeated inputs."""
    import torch
    print(f"case gdn strided tokens={tokens} chunk={chunk}", flush=True)
    rng = np.random.default_rng(tokens + chunk)
    hk, hv, d = 16, 48, 128
    width = 2 * hk * d + hv * d + 96          # padded token row
    row = (rng.standard_normal((tokens, width))).astype(np.float32)
    q = row[:, :hk * d].reshape(tokens, hk, d)
    k = row[:, hk * d:2 * hk * d].reshape(tokens, hk, d)
    v = row[:, 2 * hk * d:2 * hk * d + hv * d].reshape(tokens, hv, d)
    ld = -np.abs(rng.standard_normal((tokens, hv))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((tokens, hv))))).astype(np.float32)
    state = (rng.standard_normal((hv, d, d)) * 0.1).astype(np.float32)
    qr = np.repeat(q, 3, axis=1).reshape(-1)
    kr = np.repeat(k, 3, axis=1).reshape(-1)
    ref_state = state.reshape(-1).copy()
    ref = orc.gated_delta_sequence(qr, kr, v.reshape(-1), ld.reshape(-1), beta.reshape(-1), ref_state, tokens, hv, d, d)
    drow = torch.from_numpy(row).cuda()
    keep = [torch.from_numpy(x).cuda() for x in (ld, beta)]
    dstate = torch.from_numpy(state).cuda()
    out = torch.empty(tokens, hv, d, device="cuda")
    base = drow.data_ptr()
    hip.gated_delta_strided_device(base, base + hk * d * 4, base + 2 * hk * d * 4, width, width, keep[0].data_ptr(),
                                   keep[1].data_ptr(), dstate.data_ptr(), tokens, hv, hk, d, d, chunk, out.data_ptr())
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.cpu().numpy().reshape(-1), ref, rtol=1e-3, atol=1e-4 * float(np.abs(ref).max()))
    np.testing.assert_allclose(dstate.cpu().numpy().reshape(-1), ref_state, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("tokens,heads,key_heads,dk,dv,given,K", [(1, 48, 16, 128, 128, False, 4),
                                                                 (5, 48, 16, 128, 128, False, 4),
                                                                 (3, 4, 2, 64, 64, True, 4), (2, 8, 8, 128, 48, False, 4),
                                                                 (1, 48, 16, 128, 128, False, 3),
                                                                 (3, 4, 2, 64, 64, False, 6)])
def test_fused_mixer_core_matches_separate(hip, tokens, heads, key_heads, dk, dv, given, K):
    """ctox_hip_gdn_fused_device (conv + gates + recurrence in one launch) against
    the separate conv, gates and strided recurrence entry points (each pinned
    to the oracle by the tests above and test_gpu_layer_ops): outputs, states,
    conv windows and gates."""
    import ctypes
    import torch
    import ctox_hip
    say(f"case fused mixer tokens={tokens} heads={heads}/{key_heads} dk={dk} dv={dv} given={given} kernel={K}")
    lib = ctox_hip.load_library()
    rng = np.random.default_rng(tokens * 100 + heads + K)
    kw, vw = key_heads * dk, heads * dv
    C = 2 * kw + vw
    a_off, b_off = C + vw, C + vw + heads
    stride = b_off + heads + 3
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    proj = dev(rng.standard_normal((tokens, stride)))
    conv_w = dev(rng.standard_normal((C, K)) * 0.5)
    conv0 = rng.standard_normal((C, K)).astype(np.float32)
    a_log = dev(rng.standard_normal(heads) * 0.3)
    dt_bias = dev(rng.standard_normal(heads) * 0.3)
    state0 = (rng.standard_normal((heads, dk, dv)) * 0.1).astype(np.float32)
    ld_g = rng.uniform(-1.0, -0.05, (tokens, heads)).astype(np.float32)
    be_g = rng.uniform(0.1, 0.9, (tokens, heads)).astype(np.float32)
    # separate path
    conv_a, st_a = dev(conv0), dev(state0)
    convo = torch.empty(tokens, C, device="cuda")
    ld_a, be_a = (dev(ld_g), dev(be_g)) if given else (torch.empty(tokens, heads, device="cuda"),
                                                        torch.empty(tokens, heads, device="cuda"))
    out_a = torch.empty(tokens, heads, dv, device="cuda")
    p = lambda t: t.data_ptr()
    assert lib.ctox_hip_causal_conv_rows_device(hip.handle, p(proj), stride, p(conv_a), p(conv_w), C, K, tokens,
                                                p(convo), None) == 0
    if not given:
        assert lib.ctox_hip_gdn_gates_strided_device(hip.handle, p(proj) + 4 * a_off, p(proj) + 4 * b_off, stride,
                                                     p(a_log), p(dt_bias), tokens, heads, p(ld_a), p(be_a), None) == 0
    assert lib.ctox_hip_gated_delta_strided_device(hip.handle, p(convo), p(convo) + 4 * kw, p(convo) + 8 * kw, C, C,
                                                   p(ld_a), p(be_a), p(st_a), tokens, heads, key_heads, dk, dv, 0,
                                                   p(out_a), None) == 0
    # fused path
    conv_in, conv_out, st_b = dev(conv0), torch.zeros(C, K, device="cuda"), dev(state0)
    ld_b, be_b = (dev(ld_g), dev(be_g)) if given else (torch.empty(tokens, heads, device="cuda"),
                                                        torch.empty(tokens, heads, device="cuda"))
    out_b = torch.empty(tokens, heads, dv, device="cuda")
    st = lib.ctox_hip_gdn_fused_device(hip.handle, p(proj), stride, a_off, b_off, p(conv_w), p(conv_in), p(conv_out), K,
                                       p(a_log), p(dt_bias), p(ld_b), p(be_b), 1 if given else 0, p(st_b), tokens,
                                       heads, key_heads, dk, dv, p(out_b), None)
    assert st == 0, lib.ctox_hip_last_error()
    torch.cuda.synchronize()
    np.testing.assert_allclose(conv_out.cpu().numpy(), conv_a.cpu().numpy(), rtol=0, atol=0)
    assert np.array_equal(conv_in.cpu().numpy(), conv0)
    np.testing.assert_allclose(ld_b.cpu().numpy(), ld_a.cpu().numpy(), rtol=1e-6, atol=0)
    np.testing.assert_allclose(be_b.cpu().numpy(), be_a.cpu().numpy(), rtol=1e-6, atol=0)
    ref_o, ref_s = out_a.cpu().numpy(), st_a.cpu().numpy()
    np.testing.assert_allclose(out_b.cpu().numpy(), ref_o, rtol=1e-4, atol=1e-5 * float(np.abs(ref_o).max()))
    np.testing.assert_allclose(st_b.cpu().numpy(), ref_s, rtol=1e-4, atol=1e-5 * float(np.abs(ref_s).max()))


def test_fused_snapshots_equal_sequential_steps(hip):
    """ctox_hip_gdn_fused_snap_device: the state and conv windows after each
    row t equal those of running the fused core over the first t + 1 rows
    (in place; bit for bit from two rows on, where both run the row-block
    kernel), and the outputs are the same."""
    import torch
    import ctox_hip
    say("case fused snapshots")
    lib = ctox_hip.load_library()
    rng = np.random.default_rng(77)
    tokens, heads, key_heads, dk, dv, K = 5, 48, 16, 128, 128, 4
    kw, vw = key_heads * dk, heads * dv
    C = 2 * kw + vw
    a_off, b_off = C + vw, C + vw + heads
    stride = b_off + heads
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    p = lambda t: t.data_ptr()
    proj = dev(rng.standard_normal((tokens, stride)))
    conv_w = dev(rng.standard_normal((C, K)) * 0.5)
    conv0 = rng.standard_normal((C, K)).astype(np.float32)
    a_log = dev(rng.standard_normal(heads) * 0.3)
    dt_bias = dev(rng.standard_normal(heads) * 0.3)
    state0 = (rng.standard_normal((heads, dk, dv)) * 0.1).astype(np.float32)
    ssz, csz = heads * dk * dv, C * K
    st_in = dev(state0)
    snaps = torch.full((tokens, ssz), float("nan"), device="cuda")
    csnaps = torch.full((tokens, csz), float("nan"), device="cuda")
    conv_in = dev(conv0)
    ld, be = torch.empty(tokens, heads, device="cuda"), torch.empty(tokens, heads, device="cuda")
    out = torch.empty(tokens, heads, dv, device="cuda")
    st = lib.ctox_hip_gdn_fused_snap_device(hip.handle, p(proj), stride, a_off, b_off, p(conv_w), p(conv_in),
                                            p(csnaps), csz, K, p(a_log), p(dt_bias), p(ld), p(be), p(st_in), p(snaps),
                                            ssz, 0, tokens, heads, key_heads, dk, dv, p(out), None)
    assert st == 0, lib.ctox_hip_last_error()
    # aliasing conv windows are refused
    assert lib.ctox_hip_gdn_fused_snap_device(hip.handle, p(proj), stride, a_off, b_off, p(conv_w), p(conv_in),
                                              p(conv_in) - 4 * csz, csz, K, p(a_log), p(dt_bias), p(ld), p(be),
                                              p(st_in), p(snaps), ssz, 0, tokens, heads, key_heads, dk, dv, p(out),
                                              None) != 0
    torch.cuda.synchronize()
    assert np.array_equal(st_in.cpu().numpy(), state0)  # input untouched (other output buffer)
    for t in range(tokens):
        st_b, cin, cout = dev(state0), dev(conv0), torch.zeros(C, K, device="cuda")
        ld_b, be_b = torch.empty(t + 1, heads, device="cuda"), torch.empty(t + 1, heads, device="cuda")
        out_b = torch.empty(t + 1, heads, dv, device="cuda")
        assert lib.ctox_hip_gdn_fused_device(hip.handle, p(proj), stride, a_off, b_off, p(conv_w), p(cin), p(cout), K,
                                             p(a_log), p(dt_bias), p(ld_b), p(be_b), 0, p(st_b), t + 1, heads,
                                             key_heads, dk, dv, p(out_b), None) == 0
        torch.cuda.synchronize()
        if t == 0:
            # One row runs the one-row kernel (its key-row sums associate
            # differently): equal within float rounding.
            np.testing.assert_allclose(snaps[t].cpu().numpy(), st_b.cpu().numpy().reshape(-1), rtol=1e-5, atol=1e-6)
        else:
            assert np.array_equal(snaps[t].cpu().numpy(), st_b.cpu().numpy().reshape(-1)), t
        assert np.array_equal(csnaps[t].cpu().numpy(), cout.cpu().numpy().reshape(-1)), t
        if t == tokens - 1:
            assert np.array_equal(out.cpu().numpy(), out_b.cpu().numpy())
    # The blocked layout (the engine's): the same states, permuted.
    sl = (dv + 15) // 16

    def to_blocked(x):  # [heads][dk][dv] -> [heads][slice][ig*16 + jj][r], i = ig + 16 r, j = 16 slice + jj
        b = np.zeros((heads, sl, 16, 16, 8), np.float32)
        xx = x.reshape(heads, 8, 16, sl, 16)  # [h][r][ig][slice][jj]
        b[:] = xx.transpose(0, 3, 2, 4, 1)
        return b.reshape(-1)

    bsz = heads * sl * 2048
    st_blk = dev(to_blocked(state0))
    bsnaps = torch.full((tokens, bsz), float("nan"), device="cuda")
    csn2 = torch.full((tokens, csz), float("nan"), device="cuda")
    out2 = torch.empty(tokens, heads, dv, device="cuda")
    st = lib.ctox_hip_gdn_fused_snap_device(hip.handle, p(proj), stride, a_off, b_off, p(conv_w), p(conv_in),
                                            p(csn2), csz, K, p(a_log), p(dt_bias), p(ld), p(be), p(st_blk),
                                            p(bsnaps), bsz, 1, tokens, heads, key_heads, dk, dv, p(out2), None)
    assert st == 0, lib.ctox_hip_last_error()
    torch.cuda.synchronize()
    for t in range(tokens):
        assert np.array_equal(bsnaps[t].cpu().numpy(), to_blocked(snaps[t].cpu().numpy())), t
    assert np.array_equal(out2.cpu().numpy(), out.cpu().numpy())
    assert np.array_equal(csn2.cpu().numpy(), csnaps.cpu().numpy())
