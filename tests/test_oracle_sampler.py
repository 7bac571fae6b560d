"""Pins the oracle's Pcg32 sampler, greedy MTP verification and the
temperature rejection-sampling acceptance.

Crate cases: Q/src/sampler.rs:176-253, Q/src/engine.rs:1213-1300. The
acceptance at T > 0 has no crate counterpart (the crate's MTP is greedy
only, Q/src/engine.rs:583-590): it is pinned by the invariants of
speculative sampling -- identical draft and target laws always accept, and
the emitted token's law equals the target law (Monte Carlo).
"""
import json
import os

import numpy as np
import pytest

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "crate_goldens.json")))


def test_pcg32_reference_sequence(orc):
    # PCG-XSH-RR with the crate's increment; first outputs for seed 0 computed
    # independently here in Python integers.
    def ref(seed, n):
        s = (seed + 0x853C49E6748FEA9B) & (2 ** 64 - 1)
        out = []
        for _ in range(n + 1):
            old = s
            s = (old * 6364136223846793005 + 1442695040888963407) & (2 ** 64 - 1)
            x = (((old >> 18) ^ old) >> 27) & 0xFFFFFFFF
            r = old >> 59
            out.append(((x >> r) | (x << ((32 - r) & 31))) & 0xFFFFFFFF)
        return out[1:]
    for seed in (0, 17, 42):
        g = orc.Pcg32(seed)
        assert [g.next_u32() for _ in range(16)] == ref(seed, 16)


def test_greedy_is_argmax_and_ties_pick_later(orc):
    assert orc.sample_with_draw([-1.0, 3.0, 2.0], 0.0, 40, 0.95, 0.0) == 1
    assert orc.sample_with_draw([2.0, 2.0], 1.0, 1, 1.0, 0.0) == 1  # Q/src/sampler.rs:229-239
    assert orc.greedy_token([1.0, 5.0, 5.0, 0.0]) == 2


def test_seeded_sampling_is_deterministic(orc):
    a, b = orc.Pcg32(42), orc.Pcg32(42)
    logits = [0.1, 0.2, 0.3, 0.4]
    sa = [orc.sample_with_draw(logits, 0.8, 40, 0.95, a.next_f32()) for _ in range(32)]
    sb = [orc.sample_with_draw(logits, 0.8, 40, 0.95, b.next_f32()) for _ in range(32)]
    assert sa == sb
    assert orc.sample_with_draw([-0.5, 0.25, 1.5, 0.75], 0.8, 4, 0.9, 0.625) == \
        orc.sample_with_draw([-0.5, 0.25, 1.5, 0.75], 0.8, 4, 0.9, 0.625)


def test_sampling_law_matches_softmax(orc):
    # Closed form: with top_k = 0 and top_p = 1 the draw maps through the CDF
    # of softmax(logits / T) sorted by decreasing probability.
    logits = np.array([0.0, 1.0, -0.5, 0.3], np.float32)
    t = 0.7
    p = np.exp(logits / t - (logits / t).max())
    p /= p.sum()
    order = np.argsort(-p, kind="stable")
    cdf = np.cumsum(p[order])
    for u in np.linspace(0.0, 0.999, 200):
        want = order[np.searchsorted(cdf, u * cdf[-1] - 1e-7)]
        assert orc.sample_with_draw(logits, t, 0, 1.0, float(u)) == want


def test_draw_out_of_range_fails_closed(orc):
    import pytest
    with pytest.raises(orc.OracleError):
        orc.sample_with_draw([1.0], 1.0, 2, 1.0, 1.0)


def test_greedy_mtp_prefix_fallback_bonus(orc):
    g = GOLD["greedy_mtp"]
    tgt = [g["target"]] * 4
    nxt, ver, acc = orc.verify_greedy_mtp(g["drafts"], tgt, g["bonus"])
    assert (nxt, ver, acc) == (g["expect"]["token"], g["expect"]["verified"], g["expect"]["accepted"])
    nxt, ver, acc = orc.verify_greedy_mtp(tgt, tgt, g["bonus"])
    e = g["all_accepted_expect"]
    assert (nxt, ver, acc) == (e["token"], e["verified"], e["accepted"])


def test_mtp_accept_identical_laws_always_accept(orc):
    rng = np.random.default_rng(0)
    logits = rng.standard_normal((4, 50)).astype(np.float32)
    toks = rng.integers(0, 50, 4)
    g = orc.Pcg32(5)
    for _ in range(50):
        _, nacc = orc.mtp_accept_sample(logits, logits, logits[0], toks, 0.7, g)
        assert nacc == 4


def test_mtp_accept_output_law_equals_target(orc):
    # One draft: P(emit = x) must equal p(x) when the draft token is drawn from q.
    p_log = np.array([[1.0, 0.2, -0.3, 0.5]], np.float32)
    q_log = np.array([[-0.5, 1.2, 0.3, 0.0]], np.float32)
    t = 0.7
    p = np.exp(p_log[0] / t); p /= p.sum()
    q = np.exp(q_log[0] / t); q /= q.sum()
    rng = np.random.default_rng(1)
    g = orc.Pcg32(9)
    counts = np.zeros(4)
    n = 20000
    bonus = np.zeros(4, np.float32)
    for _ in range(n):
        d = rng.choice(4, p=q)
        nxt, nacc = orc.mtp_accept_sample(q_log, p_log, bonus, [d], t, g)
        counts[d if nacc == 1 else nxt] += 1
    assert np.max(np.abs(counts / n - p)) < 0.015


def test_mtp_accept_restricted_equals_padded_full_row(orc):
    # A restricted draft row (Q/src/engine.rs:151-200) is the full row with
    # every other token at -inf: the same draws give the same decisions.
    rng = np.random.default_rng(3)
    vocab, k = 40, 4
    ids = np.sort(rng.choice(vocab, 12, replace=False)).astype(np.uint32)
    for trial in range(30):
        dr = rng.standard_normal((k, ids.size)).astype(np.float32) * 2
        full = np.full((k, vocab), -np.inf, np.float32)
        full[:, ids] = dr
        tg = rng.standard_normal((k, vocab)).astype(np.float32) * 2
        bonus = rng.standard_normal(vocab).astype(np.float32)
        toks = ids[rng.integers(0, ids.size, k)]
        g1, g2 = orc.Pcg32(trial), orc.Pcg32(trial)
        a = orc.mtp_accept_sample(dr, tg, bonus, toks, 0.7, g1, draft_ids=ids)
        b = orc.mtp_accept_sample(full, tg, bonus, toks, 0.7, g2)
        assert a == b and g1.c.state == g2.c.state


def test_mtp_accept_restricted_output_law_equals_target(orc):
    # Drafts drawn from a restricted q still emit exactly the target law p.
    p_log = np.array([[1.0, 0.2, -0.3, 0.5, 0.1]], np.float32)
    ids = np.array([1, 3], np.uint32)
    q_log = np.array([[0.4, -0.2]], np.float32)
    t = 0.7
    p = np.exp(p_log[0] / t); p /= p.sum()
    q = np.exp(q_log[0] / t); q /= q.sum()
    rng = np.random.default_rng(2)
    g = orc.Pcg32(11)
    counts = np.zeros(5)
    n = 20000
    bonus = np.zeros(5, np.float32)
    for _ in range(n):
        d = ids[rng.choice(2, p=q)]
        nxt, nacc = orc.mtp_accept_sample(q_log, p_log, bonus, [d], t, g, draft_ids=ids)
        counts[d if nacc == 1 else nxt] += 1
    assert np.max(np.abs(counts / n - p)) < 0.015


def test_mtp_accept_restricted_rejects_noncanonical_ids(orc):
    # Q/src/decoder.rs:597-608 and Q/src/engine.rs:1387-1412: IDs must be
    # strictly increasing and inside the vocabulary.
    tg = np.zeros((1, 6), np.float32)
    for ids in ([4, 1], [1, 1], [1, 6]):
        with pytest.raises(orc.OracleError):
            orc.mtp_accept_sample(np.zeros((1, len(ids)), np.float32), tg, tg[0], [1], 0.7, orc.Pcg32(0),
                                  draft_ids=ids)
