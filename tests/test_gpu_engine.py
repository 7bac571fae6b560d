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
