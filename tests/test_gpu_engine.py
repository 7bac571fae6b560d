"""GPU parity of the device-resident decode engine against the CPU oracle of
the crate's decoder graph (oracle/decoder.py), on a small configuration of
the Qwen3.8 topology: 3 GatedDeltaNet layers and 1 full-attention layer,
head_dim 256, the MTP head with 4 drafts, paged KV with page 16, sink 16 and
recent 32 (pages demote within the test).

* Target decode: next-token logits after every step within rtol 1e-3 plus an
  absolute 1e-4 x max|logits| floor.
* Speculative steps at T = 0.7 from one seeded Pcg32 stream: the engine's
  accepted drafts and next token equal the oracle's, and the logits of a
  following plain step agree, which checks the commit (GatedDeltaNet
  restore and replay, KV truncation, MTP cache replay).
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def small_config():
    from ctox_hip.engine import EngineConfig
    return EngineConfig(256, 512, 4, 4, 2, 1, 256, 64, 2, 4, 64, 64, 4, 512, 512, 16, 16, 32, 1, 4, 1e-6, 1e7)


def close(got, want):
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-4 * float(np.abs(want).max()))


@pytest.fixture
def pair(hip):
    from ctox_hip.engine import Engine
    from oracle.decoder import OracleDecoder
    cfg = small_config()
    eng = Engine(hip, cfg, seed=3)
    orc_dec = OracleDecoder(cfg.as_dict(), eng.tensor)
    yield eng, orc_dec
    eng.close()


def test_engine_decode_matches_oracle(pair):
    eng, ref = pair
    rng = np.random.default_rng(0)
    for step in range(70):
        tok = int(rng.integers(0, 512))
        say(f"case engine decode step={step} token={tok}")
        want = ref.decode(tok)
        eng.decode(tok)
        close(eng.logits(1)[0], want)
    assert eng.position == ref.position == 70
    assert ref.caches[3].q2_tokens() > 0   # demotion happened on both sides


def test_engine_mtp_steps_match_oracle(pair):
    from oracle import oracle as orc
    eng, ref = pair
    rng = np.random.default_rng(1)
    for step in range(40):
        tok = int(rng.integers(0, 512))
        ref.decode(tok)
        eng.decode(tok)
    state0 = 0x5EED1234ABCD
    g = orc.Pcg32(0)
    g.c.state = state0
    eng.set_rng(state0)
    token = int(rng.integers(0, 512))
    accepted = []
    for step in range(8):
        say(f"case engine mtp step={step} token={token} position={ref.position}")
        nxt, acc, _ = ref.mtp_step(token, 0.7, g, 4)
        got_next, got_acc = eng.mtp_step(token, 0.7)
        assert (got_next, got_acc) == (nxt, [int(x) for x in acc]), (step, got_next, got_acc, nxt, acc)
        assert eng.position == ref.position
        accepted.append(len(acc))
        token = nxt
    say("accepted per step", accepted)
    # one plain step after the speculative ones checks every committed state
    want = ref.decode(token)
    eng.decode(token)
    close(eng.logits(1)[0], want)


def run_mtp_steps(eng, ref, rng, steps, token, T=0.7, drafts=4, tag=""):
    from oracle import oracle as orc
    state0 = 0x5EED1234ABCD
    g = orc.Pcg32(0)
    g.c.state = state0
    eng.set_rng(state0)
    accepted = []
    for step in range(steps):
        say(f"case engine mtp{tag} step={step} token={token} position={ref.position}")
        nxt, acc, _ = ref.mtp_step(token, T, g, drafts)
        got_next, got_acc = eng.mtp_step(token, T)
        assert (got_next, got_acc) == (nxt, [int(x) for x in acc]), (step, got_next, got_acc, nxt, acc)
        assert eng.position == ref.position
        accepted.append(len(acc))
        token = nxt
    say("accepted per step", accepted)
    return token


def test_engine_restricted_draft_vocab_matches_oracle(hip):
    """The restricted MTP draft head (Q/src/decoder.rs:589-627): drafts score
    only the bound draft vocabulary; acceptance uses restricted draft laws.
    Accepted drafts and next tokens equal the oracle's, and a following plain
    step's logits agree."""
    from ctox_hip.engine import Engine
    from oracle.decoder import OracleDecoder
    cfg = small_config()
    eng = Engine(hip, cfg, seed=5)
    try:
        ids = np.sort(np.random.default_rng(9).choice(512, 96, replace=False)).astype(np.uint32)
        eng.set_draft_vocab(ids)
        ref = OracleDecoder(cfg.as_dict(), eng.tensor, draft_ids=ids)
        rng = np.random.default_rng(4)
        for step in range(20):
            tok = int(rng.integers(0, 512))
            ref.decode(tok)
            eng.decode(tok)
        token = run_mtp_steps(eng, ref, rng, 8, int(rng.integers(0, 512)), tag=" restricted")
        # the draft rows are the restricted head's scores (draft logits view)
        d = eng.read(5, 4 * ids.size).reshape(4, ids.size)
        assert np.all(np.isfinite(d))
        want = ref.decode(token)
        eng.decode(token)
        close(eng.logits(1)[0], want)
    finally:
        eng.close()


def test_engine_draft_vocab_rejects_noncanonical(hip):
    import ctox_hip
    from ctox_hip.engine import Engine
    eng = Engine(hip, small_config(), seed=5)
    try:
        for bad in ([4, 1], [1, 1], [1, 512], []):
            with pytest.raises(ctox_hip.InvalidArtifact):
                eng.set_draft_vocab(bad)
        eng.set_draft_vocab([1, 2, 3])
        with pytest.raises(ctox_hip.InvalidState):
            eng.set_draft_vocab([4, 5])
    finally:
        eng.close()


def test_engine_short_recent_window_matches_oracle(hip):
    """A recent window (1 token) below the verify rows: pages are demoted only
    after the new rows are appended, in the crate's append-then-demote order.
    A zero window (the crate then appends Q2 rows to the page being filled)
    is refused."""
    import ctox_hip
    from ctox_hip.engine import Engine
    from oracle.decoder import OracleDecoder
    cfg = small_config()
    cfg.recent_tokens = 0
    with pytest.raises(ctox_hip.UnsupportedOperation):
        Engine(hip, cfg, seed=7)
    cfg.recent_tokens = 1
    cfg.sink_tokens = 0
    eng = Engine(hip, cfg, seed=7)
    try:
        ref = OracleDecoder(cfg.as_dict(), eng.tensor)
        rng = np.random.default_rng(8)
        for step in range(36):
            tok = int(rng.integers(0, 512))
            say(f"case engine recent=1 decode step={step}")
            want = ref.decode(tok)
            eng.decode(tok)
            close(eng.logits(1)[0], want)
        token = run_mtp_steps(eng, ref, rng, 4, int(rng.integers(0, 512)), tag=" recent=1")
        want = ref.decode(token)
        eng.decode(token)
        close(eng.logits(1)[0], want)
        assert ref.caches[3].q2_tokens() > 0
    finally:
        eng.close()


def _poison(eng, name):
    """Writes NaN into an engine weight vector (host-side write, then the next step reads it)."""
    import ctypes
    from ctox_hip.engine import EngineTensor, _lib, _check
    t = EngineTensor()
    _check(_lib().ctox_hip_engine_tensor(eng.handle, name.encode(), ctypes.byref(t)))
    nan = np.full(t.bytes // 4, np.nan, np.float32)
    rt = ctypes.CDLL("libamdhip64.so")
    rt.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert rt.hipMemcpy(t.data, nan.ctypes.data, t.bytes, 1) == 0


def test_engine_fails_closed_on_nonfinite_logits(hip):
    """Non-finite logits end the step with InvalidState
    (Q/src/backend/cuda_runtime.rs:10627-10632, Q/src/engine.rs:191-272):
    plain decode, and an MTP step whose draft head is poisoned."""
    import ctox_hip
    from ctox_hip.engine import Engine
    eng = Engine(hip, small_config(), seed=11)
    try:
        eng.decode(3)
        eng.decode(4)
        _poison(eng, "mtp.norm")
        with pytest.raises(ctox_hip.InvalidState):
            eng.mtp_step(5, 0.7)
    finally:
        eng.close()
    eng = Engine(hip, small_config(), seed=11)
    try:
        eng.decode(3)
        _poison(eng, "final_norm")
        with pytest.raises(ctox_hip.InvalidState):
            eng.decode(4)
    finally:
        eng.close()


def _write_vec(eng, ref, name, values):
    """Overwrites an engine weight vector on the device (a raw copy into the
    tensor: the engine refuses writes once loaded) and the oracle's copy."""
    import ctypes
    from ctox_hip.engine import EngineTensor, _lib, _check
    t = EngineTensor()
    _check(_lib().ctox_hip_engine_tensor(eng.handle, name.encode(), ctypes.byref(t)))
    v = np.ascontiguousarray(values, np.float32)
    assert v.nbytes == t.bytes
    rt = ctypes.CDLL("libamdhip64.so")
    rt.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert rt.hipMemcpy(t.data, v.ctypes.data, t.bytes, 1) == 0
    ref.w(name)["data"] = v.copy()


def sync_caches(eng, ref, kvw):
    """Adopts the engine's paged K/V bytes into the oracle after checking that
    they differ from the oracle's only where quantization of nearly equal
    inputs may: a 4-bit code or 2-bit code one step apart, or an fp16 block
    scale one unit apart (the K/V rows come from matvecs that agree within
    ~1e-6 relative, and the packer is byte-exact on identical inputs, which
    test_gpu_paged_attention checks). A differing code at a rounding boundary
    otherwise shifts later logits by up to a few 1e-3, so callers reconcile
    after every step, before differences can compound."""
    layers = list(ref.caches) + ([-1] if ref.mtp_cache is not None else [])
    flips = 0
    for l in layers:
        cache = ref.caches[l] if l >= 0 else ref.mtp_cache
        got = eng.cache_pages(l)
        want = cache.page_views()
        assert [(p[0], p[1], p[2]) for p in got] == [(p[3], p[2], p[1]) for p in want]
        for (prec, tokens, _, data), wv in zip(got, want):
            bb = 34 if prec else 18
            a = np.frombuffer(data, np.uint8).reshape(-1, bb)
            b = np.frombuffer(wv[4][:len(data)], np.uint8).reshape(-1, bb)
            sa, sb = a[:, :2].copy().view(np.uint16).astype(np.int32), b[:, :2].copy().view(np.uint16).astype(np.int32)
            assert np.all(np.abs(sa - sb) <= 1), l
            bits = 4 if prec else 2
            for sh in range(0, 8, bits):
                ca = (a[:, 2:] >> sh) & ((1 << bits) - 1)
                cb = (b[:, 2:] >> sh) & ((1 << bits) - 1)
                assert np.all(np.abs(ca.astype(np.int32) - cb) <= 1), l
            flips += int(np.sum(a != b))
        cache.load_pages(got)
    return flips


@pytest.mark.parametrize("restricted", [False, True])
def test_engine_greedy_mtp_matches_oracle(hip, restricted):
    """Temperature 0 is the crate's greedy MTP (Q/src/engine.rs:583-590,
    915-963): argmax drafts (restricted: argmax over the bound IDs), longest
    prefix equal to the target argmax tokens, then the first differing target
    token or the bonus argmax. Exact tokens against the oracle; then, with the
    final norms' weights set to -1 (every final hidden 0, so all logits tie
    and the later index wins everywhere: every draft is accepted), two fully
    accepted steps; with the weights restored, a plain step's logits check
    the committed state."""
    from ctox_hip.engine import Engine
    from oracle.decoder import OracleDecoder
    cfg = small_config()
    eng = Engine(hip, cfg, seed=13)
    try:
        ids = None
        if restricted:
            ids = np.sort(np.random.default_rng(2).choice(511, 63, replace=False)).astype(np.uint32)
            ids = np.append(ids, 511).astype(np.uint32)  # the tie winner is bound
            eng.set_draft_vocab(ids)
        ref = OracleDecoder(cfg.as_dict(), eng.tensor, draft_ids=ids)
        rng = np.random.default_rng(6)
        for step in range(20):
            tok = int(rng.integers(0, 512))
            ref.decode(tok)
            eng.decode(tok)
        kvw = 2 * cfg.num_key_value_heads * cfg.head_dim
        flips = sync_caches(eng, ref, kvw)
        token = int(rng.integers(0, 512))
        for step in range(6):
            say(f"case engine greedy mtp step={step} token={token} position={ref.position}")
            nxt, acc, _ = ref.mtp_step(token, 0.0, None, 4)
            got = eng.mtp_step(token, 0.0)
            assert got == (nxt, [int(x) for x in acc]), (step, got, nxt, acc)
            assert eng.position == ref.position
            flips += sync_caches(eng, ref, kvw)
            token = nxt
        saved = {n: ref.w(n)["data"].copy() for n in ("final_norm", "mtp.norm")}
        for n in saved:
            _write_vec(eng, ref, n, np.full(cfg.hidden_size, -1.0, np.float32))
        for step in range(2):
            say(f"case engine greedy tie step={step} token={token}")
            nxt, acc, _ = ref.mtp_step(token, 0.0, None, 4)
            assert (nxt, acc) == (511, [511] * 4), (nxt, acc)
            assert eng.mtp_step(token, 0.0) == (nxt, [511] * 4)
            assert eng.position == ref.position
            flips += sync_caches(eng, ref, kvw)
            token = nxt
        for n, v in saved.items():
            _write_vec(eng, ref, n, v)
        say(f"neighbouring-code K/V bytes adopted: {flips}")
        want = ref.decode(token)
        eng.decode(token)
        close(eng.logits(1)[0], want)
    finally:
        eng.close()


def test_engine_greedy_mtp_fails_closed(hip):
    import ctox_hip
    from ctox_hip.engine import Engine
    eng = Engine(hip, small_config(), seed=11)
    try:
        eng.decode(3)
        eng.decode(4)
        for bad in (-0.5, float("nan"), float("inf")):
            with pytest.raises(ctox_hip.InvalidArtifact):
                eng.mtp_step(5, bad)
        _poison(eng, "mtp.norm")
        with pytest.raises(ctox_hip.InvalidState):
            eng.mtp_step(5, 0.0)
    finally:
        eng.close()
    eng = Engine(hip, small_config(), seed=11)
    try:
        eng.decode(3)
        eng.decode(4)
        _poison(eng, "final_norm")
        with pytest.raises(ctox_hip.InvalidState):
            eng.mtp_step(5, 0.0)
    finally:
        eng.close()
