"""Pins the oracle's gated-delta recurrence and the decoder glue ops.

Golden vectors are the crate's own (Q/src/reference.rs:531-799), which were
emitted by the pinned Python implementation. Closed forms cover what the
goldens leave open: beta = 0 only decays the state; with decay 1, beta 1
and a unit key the delta rule writes v exactly (S^T k = v afterwards); from
a zero state one token gives o = (q^.k^) beta v / sqrt(dk).
"""
import json
import math
import os

import numpy as np
import pytest

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "crate_goldens.json")))


def test_delta_step_golden(orc):
    g = GOLD["delta_step"]
    st = np.array(g["state"], np.float32)
    out = orc.gated_delta_step(g["q"], g["k"], g["v"], g["log_decay"], g["beta"], st, g["heads"], g["key_dim"],
                               g["value_dim"])
    assert np.max(np.abs(out - g["out"])) <= g["tol"]
    assert np.max(np.abs(st - g["state_out"])) <= g["tol"]


def test_delta_sequence_golden(orc):
    g = GOLD["delta_sequence"]
    st = np.array(g["state"], np.float32)
    out = orc.gated_delta_sequence(g["q"], g["k"], g["v"], g["log_decay"], g["beta"], st, g["tokens"], g["heads"],
                                   g["key_dim"], g["value_dim"])
    assert np.max(np.abs(out - g["out"])) <= g["tol"]
    assert np.max(np.abs(st - g["state_out"])) <= g["tol"]


def test_beta_zero_only_decays(orc):
    rng = np.random.default_rng(1)
    h, dk, dv = 3, 8, 5
    st = rng.standard_normal(h * dk * dv).astype(np.float32)
    ref = st.copy()
    ld = np.array([-0.1, -0.5, -2.0], np.float32)
    orc.gated_delta_step(rng.standard_normal(h * dk), rng.standard_normal(h * dk), rng.standard_normal(h * dv),
                         ld, np.zeros(h, np.float32), st, h, dk, dv)
    want = ref.reshape(h, -1) * np.exp(ld)[:, None]
    assert np.allclose(st.reshape(h, -1), want, rtol=1e-6, atol=1e-7)


def test_unit_key_write_is_exact(orc):
    rng = np.random.default_rng(2)
    h, dk, dv = 2, 16, 8
    st = rng.standard_normal(h * dk * dv).astype(np.float32)
    k = np.zeros((h, dk), np.float32)
    k[0, 3] = 2.0  # normalised to e_3
    k[1, 7] = -0.5  # normalised to -e_7
    v = rng.standard_normal((h, dv)).astype(np.float32)
    orc.gated_delta_step(rng.standard_normal(h * dk), k, v, np.zeros(h, np.float32), np.ones(h, np.float32), st,
                         h, dk, dv)
    S = st.reshape(h, dk, dv)
    assert np.allclose(S[0, 3], v[0], atol=2e-6)
    assert np.allclose(-S[1, 7], v[1], atol=2e-6)


def test_zero_state_single_token_closed_form(orc):
    rng = np.random.default_rng(3)
    h, dk, dv = 4, 128, 128
    q = rng.standard_normal((h, dk)).astype(np.float32)
    k = rng.standard_normal((h, dk)).astype(np.float32)
    v = rng.standard_normal((h, dv)).astype(np.float32)
    beta = rng.uniform(0.1, 0.9, h).astype(np.float32)
    st = np.zeros(h * dk * dv, np.float32)
    out = orc.gated_delta_step(q, k, v, -np.ones(h, np.float32), beta, st, h, dk, dv).reshape(h, dv)
    qh = q / np.sqrt((q.astype(np.float64) ** 2).sum(1, keepdims=True) + 1e-6)
    kh = k / np.sqrt((k.astype(np.float64) ** 2).sum(1, keepdims=True) + 1e-6)
    want = (qh * kh).sum(1)[:, None] * beta[:, None] * v / math.sqrt(dk)
    assert np.allclose(out, want, rtol=1e-4, atol=1e-6)


def test_f16_state_drift_bound(orc):
    # Q/src/reference.rs:630-722
    heads, kd, vd = 2, 4, 3
    s32 = np.zeros(heads * kd * vd, np.float32)
    s16 = np.zeros(heads * kd * vd, np.uint16)
    se = ss = 0.0
    mx = 0.0
    for t in range(512):
        q = [math.sin((t * 17 + i * 11 + 1) * 0.013) for i in range(heads * kd)]
        k = [math.cos((t * 13 + i * 7 + 3) * 0.017) for i in range(heads * kd)]
        v = [0.75 * math.sin((t * 19 + i * 5 + 2) * 0.011) for i in range(heads * vd)]
        ld = [-0.01 - 0.04 * ((t + h * 3) % 5) for h in range(heads)]
        be = [0.15 + 0.15 * ((t + h) % 5) for h in range(heads)]
        a = orc.gated_delta_step(q, k, v, ld, be, s32, heads, kd, vd)
        b = orc.gated_delta_step_f16_state(q, k, v, ld, be, s16, heads, kd, vd)
        d = np.abs(a - b)
        mx = max(mx, float(d.max()))
        se += float((d.astype(np.float64) ** 2).sum())
        ss += float((a.astype(np.float64) ** 2).sum())
    assert mx < 0.01 and math.sqrt(se / ss) < 0.005


def test_norms_swiglu_golden(orc):
    g = GOLD["norms"]
    assert np.max(np.abs(orc.rms_norm_1p_weight(g["values"], 1, 4, g["weight"], 1e-6) - g["rms_norm_1p"])) <= g["tol"]
    assert np.max(np.abs(orc.swiglu(g["swiglu_gate"], g["swiglu_up"]) - g["swiglu"])) <= g["tol"]
    got = orc.rms_norm_gated(g["values"], g["gated_gate"], 1, 4, g["gated_weight"], 1e-6)
    assert np.max(np.abs(got - g["rms_norm_gated"])) <= g["tol"]


def test_rope_golden(orc):
    g = GOLD["rope"]
    q = np.array(g["q"], np.float32)
    k = np.array(g["k"], np.float32)
    orc.apply_partial_rope(q, k, 1, 1, g["head_dim"], g["rotary_dim"], g["position"], g["theta"])
    assert np.max(np.abs(q - g["q_out"])) <= g["tol"] and np.max(np.abs(k - g["k_out"])) <= g["tol"]
    assert np.array_equal(q[4:], g["q_out"][4:])


def test_conv_golden(orc):
    g = GOLD["conv"]
    st = np.array(g["state"], np.float32)
    out = orc.causal_conv_silu_update(g["input"], st, g["weight"], 2, 4)
    assert np.array_equal(st, np.array(g["state_out"], np.float32))
    assert np.max(np.abs(out - g["out"])) <= g["tol"]


def test_gqa_golden_and_sigmoid_gate(orc):
    g = GOLD["gqa"]
    out = orc.grouped_query_attention(g["q"], g["k"], g["v"], g["query_heads"], g["kv_heads"], g["query_tokens"],
                                      g["kv_tokens"], g["head_dim"], g["start"])
    assert np.max(np.abs(out - g["out"])) <= g["tol"]
    gated = out.copy()
    orc.sigmoid_gate(gated, np.zeros(12, np.float32))
    assert np.all(np.abs(gated - out * 0.5) <= 1e-7)


def test_gdn_glue(orc):
    # Q/src/decoder.rs:29-35: softplus passes through above 20
    assert orc.softplus(25.0) == 25.0
    assert abs(orc.softplus(0.0) - math.log(2.0)) < 1e-7
    ld, be = orc.gdn_gates([0.5], [0.0], [0.0], [0.25])
    assert abs(be[0] - 0.5) < 1e-7 and abs(ld[0] + math.log1p(math.exp(0.75))) < 1e-6
    r = orc.repeat_heads([1, 2, 3, 4], 2, 2, 3)
    assert list(r) == [1, 2, 1, 2, 1, 2, 3, 4, 3, 4, 3, 4]
