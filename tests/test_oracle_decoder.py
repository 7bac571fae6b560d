"""Pins oracle/decoder.py (the config-5 oracle of the device engine) with the
crate's own decoder fixture, Q/src/decoder.rs:1505-2014
(`mmap_graph_executes_embedding_mlp_norm_and_lm_head`).

The fixture: hidden 64, one layer carrying both a full-attention and a
GatedDeltaNet mixer, every quantized matrix a constant-valued Q2_B64 matrix
(`recovered_matrix`, :1505-1531) with unit s_in / s_out, norm weights 0
(so (1 + w) = 1), q/k norm weights 0, conv weights [0, 1] per channel,
A_log = dt_bias = 0, gated-norm weight 1. The crate's assertions are kept
with their tolerances:

* embedding(0) is 0.5 everywhere (1e-6); token 2 is out of range;
* the full-attention residual of an all-ones hidden at position 0 is
  1 + 2 n sigmoid(n), n = (1 + 1e-6)^-1/2 (2e-4), one cached token, and the
  wrong position is refused;
* the GatedDeltaNet residual is finite and repeats after a state reset, and
  its state takes 9216 bytes (recurrent 2 x 32 x 32 f32 + conv 128 x 2 f32);
* the MLP residual of all ones is 1 + silu(n) * 2n (2e-4);
* the two LM-head logits are equal (1e-6); the restricted head over [1]
  returns exactly logits[1]; [1, 1] and [2] are refused;
* one-layer target decodes (GatedDeltaNet and full attention) give finite
  logits and repeat after a reset; the MTP draft is finite, takes one MTP
  cache entry and repeats after a reset;
* executor bookkeeping: the MTP cache always holds position - 1 entries
  through prefill, decode and every speculative commit (:1925-1960 states
  positions 2 / 1, 4 / 3 and 5 / 4).

The fused matrices are built the way the engine fuses them (row
concatenation of the members, one shared s_in), so the same tensor
provider drives the oracle exactly as the GPU parity tests do.
"""
import copy

import numpy as np
import pytest

HIDDEN = 64
HEAD_DIM, QH, KVH = 32, 2, 1
LKH, LVH, LKD, LVD, LK = 1, 2, 32, 32, 2


def q2_matrix(orc, rows, cols, value):
    block = orc.q2_quantize([value] * 64)
    return block * (rows * (cols // 64))


def fixture_tensors(orc):
    """The crate fixture's tensors under the engine's fused names."""
    one16 = lambda n: np.ones(n, np.float16).view(np.uint8)
    t = {}

    def mat(name, parts, cols):
        data = b"".join(q2_matrix(orc, r, cols, v) for r, v in parts)
        rows = sum(r for r, _ in parts)
        t[name] = {"kind": "quant", "dtype": orc.Q2B64, "rows": rows, "cols": cols, "data": data,
                   "s_in": one16(cols), "s_out": one16(rows)}

    def vec(name, values):
        t[name] = {"kind": "f32", "data": np.asarray(values, np.float32)}

    qw, kvw = QH * HEAD_DIM, KVH * HEAD_DIM
    lkw, lvw = LKH * LKD, LVH * LVD
    conv = 2 * lkw + lvw
    mat("embed", [(2, 0.5)], HIDDEN)
    for p in ("L0", "mtp"):
        mat(f"{p}.qkv", [(2 * qw, 1 / HIDDEN), (kvw, 1 / HIDDEN), (kvw, (2 if p == "L0" else 1) / HIDDEN)], HIDDEN)
        mat(f"{p}.o", [(HIDDEN, 1 / qw)], qw)
        mat(f"{p}.gate_up", [(HIDDEN, 1 / HIDDEN), (HIDDEN, 2 / HIDDEN if p == "L0" else 1 / HIDDEN)], HIDDEN)
        mat(f"{p}.down", [(HIDDEN, 1 / HIDDEN)], HIDDEN)
        vec(f"{p}.q_norm", np.zeros(HEAD_DIM))
        vec(f"{p}.k_norm", np.zeros(HEAD_DIM))
        vec(f"{p}.mlp_norm", np.zeros(HIDDEN))
    vec("L0.norm", np.zeros(HIDDEN))
    vec("mtp.attn_norm", np.zeros(HIDDEN))
    mat("L0.in", [(conv, 1 / HIDDEN), (lvw, 1 / HIDDEN), (LVH, 1 / HIDDEN), (LVH, 1 / HIDDEN)], HIDDEN)
    vec("L0.conv_w", np.tile([0.0, 1.0], conv))
    vec("L0.a_log", np.zeros(LVH))
    vec("L0.dt_bias", np.zeros(LVH))
    vec("L0.gnorm", np.ones(LVD))
    mat("L0.out", [(HIDDEN, 1 / lvw)], lvw)
    mat("lm_head", [(2, 1 / HIDDEN)], HIDDEN)
    vec("final_norm", np.zeros(HIDDEN))
    mat("mtp.fc", [(HIDDEN, 1 / (2 * HIDDEN))], 2 * HIDDEN)
    for n in ("mtp.norm", "mtp.norm_emb", "mtp.norm_hid"):
        vec(n, np.zeros(HIDDEN))
    return t


def config(layers=1, interval=4, mtp=1, max_tokens=12):
    return {"hidden_size": HIDDEN, "intermediate_size": HIDDEN, "num_hidden_layers": layers,
            "full_attention_interval": interval, "num_attention_heads": QH, "num_key_value_heads": KVH,
            "head_dim": HEAD_DIM, "rotary_dim": 16, "linear_num_key_heads": LKH, "linear_num_value_heads": LVH,
            "linear_key_head_dim": LKD, "linear_value_head_dim": LVD, "linear_conv_kernel_dim": LK,
            "vocab_size": 2, "max_tokens": max_tokens, "page_tokens": 16, "sink_tokens": 0,
            "recent_tokens": max_tokens, "mtp_layers": mtp, "draft_tokens": 4, "rms_norm_epsilon": 1e-6,
            "rope_theta": 10000.0}


@pytest.fixture
def tensors(orc):
    return fixture_tensors(orc)


def decoder(tensors, draft_ids=None, **kw):
    from oracle.decoder import OracleDecoder
    return OracleDecoder(config(**kw), lambda n: tensors[n], draft_ids=draft_ids)


def test_embedding(orc, tensors):
    dec = decoder(tensors)
    e = dec.embedding(0)
    assert e.shape == (HIDDEN,) and np.all(np.abs(e - 0.5) < 1e-6)
    with pytest.raises(orc.OracleError):
        dec.embedding(2)


def test_full_attention_residual_closed_form(orc, tensors):
    dec = decoder(tensors, interval=1)
    cache = dec.caches[0]
    ones = np.ones(HIDDEN, np.float32)
    out = dec.attention_residual("L0", ones, 0, cache)
    n = np.float32(1.0 + 1e-6) ** np.float32(-0.5)
    expected = 1.0 + 2.0 * n / (1.0 + np.exp(-n))
    assert np.all(np.abs(out - expected) < 2e-4)
    assert cache.tokens() == 1
    with pytest.raises(orc.OracleError):
        dec.attention_residual("L0", ones, 2, cache)


def test_linear_attention_residual_finite_and_repeatable(tensors):
    dec = decoder(tensors)
    # decoder.rs:1800: LinearAttentionState::allocated_bytes() == 9216
    assert (dec.gdn_state[0].nbytes + dec.conv_state[0].nbytes) == 9216
    ones = np.ones(HIDDEN, np.float32)
    fresh = (copy.deepcopy(dec.gdn_state), copy.deepcopy(dec.conv_state))
    out = ones + dec.gdn(0, dec.norm(ones, "L0.norm"))
    assert out.shape == (HIDDEN,) and np.all(np.isfinite(out))
    dec.gdn_state, dec.conv_state = copy.deepcopy(fresh[0]), copy.deepcopy(fresh[1])
    again = ones + dec.gdn(0, dec.norm(ones, "L0.norm"))
    np.testing.assert_array_equal(out, again)


def test_mlp_residual_closed_form(tensors):
    dec = decoder(tensors)
    ones = np.ones(HIDDEN, np.float32)
    out = dec.mlp("L0", ones)
    inv = (1.0 + 1e-6) ** -0.5
    gate, up = inv, 2.0 * inv
    expected = 1.0 + gate / (1.0 + np.exp(-gate)) * up
    assert np.all(np.abs(out - expected) < 2e-4)


def test_lm_head_and_restricted_head(orc, tensors):
    dec = decoder(tensors)
    out = dec.mlp("L0", np.ones(HIDDEN, np.float32))
    fin = dec.norm(out, "final_norm")
    logits = dec.matvec("lm_head", fin)
    assert logits.shape == (2,) and np.all(np.isfinite(logits))
    assert abs(float(logits[0] - logits[1])) < 1e-6
    r = dec.restricted_logits(fin, [1])
    assert r.tolist() == [logits[1]]  # decoder.rs:1852-1862: exact equality
    for bad in ([1, 1], [2]):
        with pytest.raises(orc.OracleError):
            dec.restricted_logits(fin, bad)


def test_one_layer_target_decodes_repeat(tensors):
    for interval in (4, 1):  # GatedDeltaNet, then full attention
        dec = decoder(tensors, interval=interval, mtp=0)
        logits, fin = dec.target_step(0)
        assert logits.shape == (2,) and np.all(np.isfinite(logits)) and dec.position == 1
        dec2 = decoder(tensors, interval=interval, mtp=0)
        np.testing.assert_array_equal(dec2.target_step(0)[0], logits)


def test_mtp_draft_finite_and_repeatable(orc, tensors):
    dec = decoder(tensors, interval=1)
    _, fin = dec.target_step(0)
    g, lg = dec.mtp(0, fin, 1, retain=False)
    assert g.shape == (HIDDEN,) and lg.shape == (2,) and np.all(np.isfinite(lg))
    assert dec.mtp_cache.tokens() == 1
    with pytest.raises(orc.OracleError):  # decoder.rs:1893-1902: position 2 is refused
        dec.mtp(0, fin, 3, retain=False)
    dec2 = decoder(tensors, interval=1)
    _, fin2 = dec2.target_step(0)
    g2, lg2 = dec2.mtp(0, fin2, 1, retain=False)
    np.testing.assert_array_equal(lg2, lg)
    np.testing.assert_array_equal(g2, g)


@pytest.mark.parametrize("draft_ids", [None, [0, 1], [1]])
def test_speculative_bookkeeping(orc, tensors, draft_ids):
    """Prefill, decode and speculative commits keep the MTP cache at
    position - 1 entries (decoder.rs:1925-1960); every committed step adds
    accepted + 1 positions. With equal draft and target laws (the fixture's
    two logits are equal) every full-vocabulary draft is accepted."""
    dec = decoder(tensors, draft_ids=draft_ids, max_tokens=32)
    dec.decode(0)
    assert dec.position == 1 and dec.mtp_cache.tokens() == 0
    dec.decode(1)
    assert dec.position == 2 and dec.mtp_cache.tokens() == 1
    g = orc.Pcg32(7)
    token = 0
    for _ in range(4):
        p = dec.position
        nxt, acc, info = dec.mtp_step(token, 0.7, g, 4)
        assert dec.position == p + len(acc) + 1
        assert dec.mtp_cache.tokens() == dec.position - 1
        assert all(0 <= d < 2 for d in info["drafts"]) and 0 <= nxt < 2
        if draft_ids is None:
            assert len(acc) == 4
        if draft_ids == [1]:
            assert all(d == 1 for d in info["drafts"])
            assert all(lg.shape == (1,) for lg in info["draft_logits"])
        token = nxt


@pytest.mark.parametrize("draft_ids", [None, [1]])
def test_greedy_speculative_step_is_verify_greedy_mtp(orc, tensors, draft_ids):
    """Temperature 0 is the crate's greedy MTP (engine.rs:583-590, 915-963):
    every draft is its row's argmax and the decision is verify_greedy_mtp's
    (pinned by the crate's accept / fallback / bonus cases). The fixture's two
    logits are equal, so the later index wins every argmax: all drafts are 1,
    all accepted, the next token is the bonus argmax 1. The generator is not
    consumed."""
    dec = decoder(tensors, draft_ids=draft_ids, max_tokens=32)
    dec.decode(0)
    dec.decode(1)
    g = orc.Pcg32(7)
    before = orc.Pcg32(7).next_u32()
    p = dec.position
    nxt, acc, info = dec.mtp_step(1, 0.0, g, 4)
    assert info["drafts"] == [1, 1, 1, 1] and acc == [1, 1, 1, 1] and nxt == 1
    assert dec.position == p + 5 and dec.mtp_cache.tokens() == dec.position - 1
    assert g.next_u32() == before
    if draft_ids is None:
        ref = orc.verify_greedy_mtp(np.stack(info["draft_logits"]), np.stack(info["target_logits"][:4]),
                                    info["target_logits"][4])
        assert ref == (nxt, 4, acc)


def test_verify_greedy_tokens_equals_full_logits_branch(orc):
    """The compact branch used by the greedy step equals verify_greedy_mtp's
    full-logits branch (pinned by the crate's cases) on random rows with
    planted agreements."""
    from oracle.decoder import verify_greedy_tokens
    rng = np.random.default_rng(3)
    for case in range(200):
        k, vocab = int(rng.integers(1, 6)), int(rng.integers(2, 9))
        draft = rng.normal(size=(k, vocab)).astype(np.float32)
        target = rng.normal(size=(k, vocab)).astype(np.float32)
        for i in range(k):  # make a prefix of the drafts agree, of random length
            if rng.random() < 0.7:
                target[i] = draft[i]
        bonus = rng.normal(size=vocab).astype(np.float32)
        nxt, ver, acc = orc.verify_greedy_mtp(draft, target, bonus)
        d = [orc.greedy_token(r) for r in draft]
        t = [orc.greedy_token(r) for r in list(target) + [bonus]]
        assert verify_greedy_tokens(d, t) == (nxt, len(acc))
        assert acc == d[:len(acc)]


def test_speculative_commit_equals_plain_decoding(orc, tmp_path):
    """The speculative flow at T = 0.7 (no crate counterpart) against the
    property its commit must have: after three speculative steps, a twin that
    plain-decodes the committed tokens reaches the same position and the same
    next logits (a random-weight model written as a `.ctoxq` file: 3
    GatedDeltaNet layers and one full-attention layer, MTP k = 4)."""
    from artifact_model import write_artifact
    from test_artifact_loader import small_config
    from oracle.decoder import ArtifactTensors, OracleDecoder
    cfg = small_config()
    path = tmp_path / "model.ctoxq"
    write_artifact(path, cfg, seed=5)
    spec = OracleDecoder(cfg.as_dict(), ArtifactTensors(path, cfg.as_dict()))
    plain = OracleDecoder(cfg.as_dict(), ArtifactTensors(path, cfg.as_dict()))
    rng = np.random.default_rng(3)
    for _ in range(6):
        tok = int(rng.integers(0, cfg.vocab_size))
        spec.decode(tok)
        plain.decode(tok)
    g = orc.Pcg32(21)
    token = int(rng.integers(0, cfg.vocab_size))
    committed = []
    for _ in range(3):
        nxt, acc, _ = spec.mtp_step(token, 0.7, g, 4)
        committed += [token] + [int(x) for x in acc]
        token = nxt
    for t in committed:
        plain.decode(t)
    assert spec.position == plain.position == 6 + len(committed)
    a, b = spec.decode(token), plain.decode(token)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6 * float(np.abs(b).max()))
