"""The decode engine loaded from a `.ctoxq` artifact (ctox_hip.loader) against
the oracle decoder reading the same file on its own (ArtifactTensors).

The artifact carries the crate's tensor names and a mix of packed dtypes:
pure-Q2 fused groups (gate/up, q/k/v), Q4 down projections, Q4 / Q2 / mixed
members of one GatedDeltaNet input group (Q2 rows widened on load), a Q2
embedding and mixed LM head, MTP fc and MTP gate. Bar: logits of 24 plain
steps within rtol 1e-3 plus 1e-4 x max|logits|; MTP steps at T = 0.7 and
greedy (T = 0) with exactly the oracle's accepted drafts and next tokens,
with the full and with a restricted draft head.
"""
import sys

import numpy as np
import pytest

from artifact_model import write_artifact
from test_artifact_loader import MIXED, small_config

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def close(got, want):
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-4 * float(np.abs(want).max()))


@pytest.mark.parametrize("temperature", [0.7, 0.0])
@pytest.mark.parametrize("draft_ids", [None, list(range(0, 512, 3))])
def test_engine_from_artifact_matches_oracle(hip, tmp_path, draft_ids, temperature):
    from oracle import oracle as orc
    from oracle.decoder import ArtifactTensors, OracleDecoder
    from ctox_hip.loader import load_engine
    cfg = small_config()
    path = tmp_path / "model.ctoxq"
    write_artifact(path, cfg, MIXED, seed=11)
    say(f"case engine artifact load draft_ids={'none' if draft_ids is None else len(draft_ids)}")
    eng = load_engine(hip, path, cfg, draft_ids=draft_ids)
    try:
        for name, dtype in (("L0.in", orc.Q4B64), ("L1.gate_up", orc.Q2B64), ("L3.qkv", orc.Q2B64),
                            ("L2.down", orc.Q4B64), ("embed", orc.Q2B64), ("lm_head", orc.Q4B64)):
            assert eng.tensor_info(name)["dtype"] == dtype, name
        ref = OracleDecoder(cfg.as_dict(), ArtifactTensors(path, cfg.as_dict()), draft_ids=draft_ids)
        rng = np.random.default_rng(0)
        for step in range(24):
            tok = int(rng.integers(0, cfg.vocab_size))
            say(f"case engine artifact decode step={step} token={tok}")
            want = ref.decode(tok)
            eng.decode(tok)
            close(eng.logits(1)[0], want)
        state0 = 0x1234567
        g = orc.Pcg32(0)
        g.c.state = state0
        eng.set_rng(state0)
        token = int(rng.integers(0, cfg.vocab_size))
        for step in range(6):
            say(f"case engine artifact mtp step={step} token={token}")
            nxt, acc, _ = ref.mtp_step(token, temperature, g, 4)
            got = eng.mtp_step(token, temperature)
            assert got == (nxt, [int(x) for x in acc]), (step, got, nxt, acc)
            token = nxt
        want = ref.decode(token)
        eng.decode(token)
        close(eng.logits(1)[0], want)
    finally:
        eng.close()


def test_engine_refuses_steps_while_loading(hip):
    from ctox_hip import InvalidState, ShapeError
    from ctox_hip.engine import Engine
    cfg = small_config()
    eng = Engine(hip, cfg, seed=1)
    try:
        ones = np.ones(cfg.hidden_size, np.float32)
        eng.write("final_norm", 0, 0, ones)
        with pytest.raises(InvalidState):
            eng.decode(1)
        with pytest.raises(ShapeError):  # past the end of the tensor
            eng.write("final_norm", 0, 4, ones)
        eng.finish_load()
        eng.decode(1)
        assert np.all(np.isfinite(eng.logits(1)))
        with pytest.raises(InvalidState):  # no writes into a running engine
            eng.write("final_norm", 0, 0, ones)
    finally:
        eng.close()
