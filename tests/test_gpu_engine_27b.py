"""The decode engine at Qwen3.8-27B layer dimensions.

* Oracle parity at real layer shapes with fewer layers: hidden 5120, 24 query
  / 4 KV heads of 256, 48 value / 16 key GatedDeltaNet heads of 128,
  intermediate 17408, vocab 151936, page 16, three GatedDeltaNet layers and
  one full-attention layer, a 2048-token context filled on the device and
  loaded into the oracle page by page. Plain steps' logits within rtol 1e-3
  plus 1e-4 x max|logits|; MTP k = 4 steps at T = 0.7 with exactly the
  oracle's accepted drafts and next tokens, then greedy (T = 0) MTP steps
  with exactly the oracle's tokens.
* Properties of the full 64-layer engine at 4096- and 32768-token contexts
  (config 5's stated context): every
  step's logits are finite, and after MTP commits the engine is in the state
  plain decoding of the committed tokens reaches (the next step's logits and
  the following speculative step's first draft row agree).
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def close(got, want):
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-4 * float(np.abs(want).max()))


def config27(layers, max_tokens):
    from ctox_hip.engine import EngineConfig
    c = EngineConfig.qwen38_27b(max_tokens=max_tokens, vocab=151936, page_tokens=16, drafts=4)
    c.num_hidden_layers = layers
    return c


@pytest.mark.timeout(900)
def test_engine_27b_layer_dims_match_oracle(hip):
    from oracle import oracle as orc
    from oracle.decoder import OracleDecoder
    from ctox_hip.engine import Engine
    cfg = config27(4, 2048 + 64)
    say("case engine27 create (4 layers, 27B dims)")
    eng = Engine(hip, cfg, seed=21)
    try:
        eng.fill_context(2048, seed=3)
        ref = OracleDecoder(cfg.as_dict(), eng.tensor)
        ref.load_context(eng.cache_pages, eng.position, eng.read(2, cfg.hidden_size))
        rng = np.random.default_rng(5)
        for step in range(2):
            tok = int(rng.integers(0, cfg.vocab_size))
            say(f"case engine27 decode step={step} token={tok}")
            want = ref.decode(tok)
            eng.decode(tok)
            close(eng.logits(1)[0], want)
        state0 = 0xC0FFEE
        g = orc.Pcg32(0)
        g.c.state = state0
        eng.set_rng(state0)
        token = int(rng.integers(0, cfg.vocab_size))
        for step in range(2):
            say(f"case engine27 mtp step={step} token={token} position={ref.position}")
            nxt, acc, _ = ref.mtp_step(token, 0.7, g, 4)
            got = eng.mtp_step(token, 0.7)
            assert got == (nxt, [int(x) for x in acc]), (step, got, nxt, acc)
            assert eng.position == ref.position
            token = nxt
        for step in range(2):  # the crate's greedy MTP (engine.rs:583-590, 915-963)
            say(f"case engine27 greedy mtp step={step} token={token} position={ref.position}")
            nxt, acc, _ = ref.mtp_step(token, 0.0, None, 4)
            got = eng.mtp_step(token, 0.0)
            assert got == (nxt, [int(x) for x in acc]), (step, got, nxt, acc)
            assert eng.position == ref.position
            token = nxt
        say("case engine27 final decode")
        want = ref.decode(token)
        eng.decode(token)
        close(eng.logits(1)[0], want)
    finally:
        eng.close()


@pytest.mark.timeout(900)
@pytest.mark.parametrize("context", [4096, 32768])
def test_engine_27b_full_depth_commit_equals_plain_decode(hip, context):
    from ctox_hip.engine import Engine
    cfg = config27(64, context + 64)
    say(f"case engine27 full depth context={context}: create two engines")
    spec = Engine(hip, cfg, seed=2)
    plain = Engine(hip, cfg, seed=2)
    try:
        for e in (spec, plain):
            e.fill_context(context, seed=9)
        spec.set_rng(12345)
        token = 17
        committed = []
        for step in range(4):
            say(f"case engine27 full depth mtp step={step}")
            nxt, acc = spec.mtp_step(token, 0.7)
            committed += [token] + acc
            assert np.all(np.isfinite(spec.logits(5)))
            token = nxt
        say(f"case engine27 full depth plain replay of {len(committed)} tokens")
        for t in committed:
            plain.decode(t)
            assert np.all(np.isfinite(plain.logits(1)[0]))
        assert plain.position == spec.position
        spec.decode(token)
        plain.decode(token)
        close(spec.logits(1)[0], plain.logits(1)[0])
        # The MTP caches agree too: the first draft row of the same speculative
        # step (it depends only on the MTP cache, the token and the previous
        # hidden) is the same within tolerance. Sampled tokens are not
        # compared: the caches hold Q4 codes of K/V computed on different
        # kernel paths, so a value at a rounding boundary may take the
        # neighbouring code, and a 151936-way cumulative draw can then pick
        # the next index.
        spec.set_rng(0x9E3779B97F4A7C15)
        plain.set_rng(0x9E3779B97F4A7C15)
        spec.mtp_step(5, 0.7)
        plain.mtp_step(5, 0.7)
        v = cfg.vocab_size
        close(spec.read(5, v), plain.read(5, v))
    finally:
        spec.close()
        plain.close()


@pytest.mark.timeout(900)
def test_engine_27b_next_norm_staging_matches_separate_staging(hip, monkeypatch):
    """The speculative verify pass with each residual producer (o_proj,
    out_proj, down at 5 rows) staging the next (1 + w) RMS-normed projection
    itself, 1 / rms applied by the consumer, against the same engine with the
    norm staged by its own launch (CTOX_NEXT_NORM=0): the 5 verify logit rows
    of two speculative steps agree within the plain-step tolerance, and so do
    the accepted drafts and next tokens."""
    from ctox_hip.engine import Engine
    cfg = config27(4, 1024 + 64)
    engines = []
    try:
        for flag in ("0", "1"):
            monkeypatch.setenv("CTOX_NEXT_NORM", flag)
            say(f"case engine27 next-norm staging={flag}: create")
            e = Engine(hip, cfg, seed=33)
            e.fill_context(1024, seed=4)
            e.set_rng(777)
            engines.append(e)
        token = 321
        for step in range(2):
            say(f"case engine27 next-norm mtp step={step} token={token}")
            got = [e.mtp_step(token, 0.7) for e in engines]
            close(engines[1].logits(5), engines[0].logits(5))
            assert got[0] == got[1], (step, got)
            token = got[0][0]
    finally:
        for e in engines:
            e.close()
