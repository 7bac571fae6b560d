"""Closed-form pins for three compositions of the oracle that the crate's own
tests leave open:

* the GatedDeltaNet layer (`OracleDecoder.gdn`, Q/src/decoder.rs:806-938):
  the crate's fixture only asserts a finite, repeatable residual
  (:1788-1800). Here its first-token residual is derived by hand from the
  fixture's constants, and a variant fixture with distinct values in every
  row block of the in-projection (q, k, v, z, a, b), a two-tap convolution
  and a head-signed out-projection is checked over two tokens against the
  rank-2 closed form of the delta rule. Each plausible slip (a/b swapped,
  q/k swapped, z taken from the value rows, conv taps reversed, heads
  swapped in the out-projection) is shown to move that closed form far
  beyond the tolerance, so the oracle cannot pass with it;
* the MTP input order (`OracleDecoder.mtp_fc`, :1027-1036): an fc whose
  embedding half and hidden half differ, under different norm weights;
* the top-k / top-p truncation of `sample_with_draw` (Q/src/sampler.rs:
  65-143): brute force over small vocabularies, with the truncated law
  built by hand in float64 and the draw swept over a fine grid.

and, with no crate counterpart (the crate's MTP is greedy), the T > 0
rejection-sampling accept (`mtp_accept_sample`): decisions the definition
fixes (accept iff u q(d) < p(d) for the next draw, the residual
max(p - q, 0), the order in which draws are consumed).

The expected values are derived from the crate's definitions, never from
the oracle's code: softplus/sigmoid/SiLU and the rank-1 key structure of the
fixture (every key is a constant-per-row vector) turn the recurrence into a
handful of scalars.
"""
import math

import numpy as np
import pytest

from test_oracle_decoder import HIDDEN, LKD, LVD, LVH, config, fixture_tensors

EPS = 1e-6      # rms_norm_epsilon of the fixture
L2_EPS = 1e-6   # reference.rs L2_EPSILON of the q/k normalisation


def silu(x):
    return x / (1.0 + np.exp(-x))


def sigmoid(x):
    return 1.0 / (1.0 + math.exp(-x))


def softplus(x):
    return x if x > 20.0 else math.log1p(math.exp(x))


def decoder_with(tensors, **kw):
    from oracle.decoder import OracleDecoder
    return OracleDecoder(config(**kw), lambda n: tensors[n])


# ----------------------------------------------------------- GatedDeltaNet
def test_gdn_first_token_closed_form_on_crate_fixture(tensors_crate):
    """Every in-projection row is 1/64 and x = n*1 (n = (1 + 1e-6)^-1/2), so
    mixed = z = a = b = n; conv taps [0, 1] give s = silu(n) everywhere; with
    a zero state the delta rule writes beta*v along k^, so each head's core
    is the constant c = (q^.k^) beta s / sqrt(32) with q^.k^ = 32 s^2 /
    (32 s^2 + 1e-6) and beta = sigmoid(n); the gated norm turns it into
    c / sqrt(c^2 + eps) * silu(n), and the out-projection (1/64 over 64
    columns) averages it: residual = 1 + c / sqrt(c^2 + eps) * silu(n)."""
    dec = decoder_with(tensors_crate)
    ones = np.ones(HIDDEN, np.float32)
    out = ones + dec.gdn(0, dec.norm(ones, "L0.norm"))
    n = (1.0 + EPS) ** -0.5
    s = float(silu(n))
    qk = 32 * s * s / (32 * s * s + L2_EPS)
    c = qk * sigmoid(n) * s / math.sqrt(32)
    expected = 1.0 + c / math.sqrt(c * c + EPS) * s
    assert np.all(np.abs(out - expected) < 2e-4), (out[:4], expected)


# Variant fixture: per-row constants (units of 1/64, fp16-exact) in every
# row block of L0.in, so each block's position in the fused rows matters.
Q_ROWS = [((r % 4) - 1.5) * 0.5 for r in range(LKD)]
K_ROWS = [((r * 3) % 5 - 2.5) * 0.5 for r in range(LKD)]
V_ROWS = [(((r * 7) % 9) - 4) * 0.25 for r in range(LVH * LVD)]
Z_ROWS = [(((r * 5) % 7) - 3) * 0.5 + 0.25 for r in range(LVH * LVD)]
A_ROWS = [1.0, -2.0]
B_ROWS = [2.0, -0.5]
CONV_TAPS = (0.5, 1.0)   # (previous token, current token), per channel


def variant_tensors(orc):
    t = fixture_tensors(orc)
    one16 = lambda k: np.ones(k, np.float16).view(np.uint8)
    rows = Q_ROWS + K_ROWS + V_ROWS + Z_ROWS + A_ROWS + B_ROWS
    data = b"".join(orc.q2_quantize([v / HIDDEN] * HIDDEN) for v in rows)
    t["L0.in"] = {"kind": "quant", "dtype": orc.Q2B64, "rows": len(rows), "cols": HIDDEN, "data": data,
                  "s_in": one16(HIDDEN), "s_out": one16(len(rows))}
    conv_ch = 2 * LKD + LVH * LVD
    t["L0.conv_w"] = {"kind": "f32", "data": np.tile(np.asarray(CONV_TAPS, np.float32), conv_ch)}
    # out-projection: head 0's columns weigh +1/64, head 1's -1/(3*64).
    lvw = LVH * LVD
    row = orc.q2_quantize([1.0 / lvw] * LVD + [-1.0 / (3 * lvw)] * LVD)
    t["L0.out"] = {"kind": "quant", "dtype": orc.Q2B64, "rows": HIDDEN, "cols": lvw, "data": row * HIDDEN,
                   "s_in": one16(lvw), "s_out": one16(HIDDEN)}
    return t


def gdn_closed_form(q_rows, k_rows, v_rows, z_rows, a_rows, b_rows, taps, out_signs=(1.0, -1.0 / 3)):
    """The layer output (before the residual) of two tokens with input
    x = n*1 and a zero state, from the crate's definitions:

    projection row r gives m_r = c_r n; the conv of token t is
    silu(w_new m + w_old m_prev) (m_prev = 0 for the first token); the one
    key head is repeated to both value heads; beta_h = sigmoid(b_h n),
    g_h = exp(-softplus(a_h n)) (A_log = dt_bias = 0). With S0 = 0 the state
    after token 1 is k1^ u1^T, u1 = beta v1 (rank 1), so token 2 sees
    memory = g (k1^.k2^) u1, delta = beta (v2 - memory), and the state
    g k1^ u1^T + k2^ delta^T. Read-outs: o1 = (q1^.k1^) u1 / sqrt(dk),
    o2 = (g (q2^.k1^) u1 + (q2^.k2^) delta) / sqrt(dk). The gated norm
    (weight 1) and the out-projection (a head's columns all weigh
    out_signs[h] / 64) follow."""
    n = (1.0 + EPS) ** -0.5
    m = {key: np.asarray(rows, np.float64) * n for key, rows in
         (("q", q_rows), ("k", k_rows), ("v", v_rows))}
    w_old, w_new = taps
    conv = [{key: silu(w_new * val) for key, val in m.items()},
            {key: silu(w_new * val + w_old * val) for key, val in m.items()}]
    unit = lambda x: x / math.sqrt(float(x @ x) + L2_EPS)
    q1, k1 = unit(conv[0]["q"]), unit(conv[0]["k"])
    q2, k2 = unit(conv[1]["q"]), unit(conv[1]["k"])
    z = silu(np.asarray(z_rows, np.float64) * n)
    outs, cores = [], []
    for tok in range(2):
        total, core = 0.0, []
        for h in range(LVH):
            beta = sigmoid(b_rows[h] * n)
            g = math.exp(-softplus(a_rows[h] * n))
            v1 = conv[0]["v"][h * LVD:(h + 1) * LVD]
            v2 = conv[1]["v"][h * LVD:(h + 1) * LVD]
            u1 = beta * v1
            if tok == 0:
                o = float(q1 @ k1) * u1 / math.sqrt(LKD)
            else:
                delta = beta * (v2 - g * float(k1 @ k2) * u1)
                o = (g * float(q2 @ k1) * u1 + float(q2 @ k2) * delta) / math.sqrt(LKD)
            y = o / math.sqrt(float(o @ o) / LVD + EPS) * z[h * LVD:(h + 1) * LVD]
            total += out_signs[h] * float(y.sum()) / (LVH * LVD)
            core.append(y)
        outs.append(total)
        cores.append(np.concatenate(core))
    return np.array(outs), np.array(cores)


def test_gdn_two_token_closed_form_distinct_blocks(orc):
    t = variant_tensors(orc)
    dec = decoder_with(t)
    x = dec.norm(np.ones(HIDDEN, np.float32), "L0.norm")
    cores, got = [], []
    for _ in range(2):
        saved = (dec.gdn_state[0].copy(), dec.conv_state[0].copy())
        cores.append(dec.gdn_core(0, x))
        dec.gdn_state[0][:], dec.conv_state[0][:] = saved
        got.append(dec.gdn(0, x))
    cores, got = np.array(cores), np.array(got)
    assert got.shape == (2, HIDDEN) and cores.shape == (2, LVH * LVD)
    # Every output row is the same dot product: one scalar per token.
    np.testing.assert_allclose(got, np.repeat(got[:, :1], HIDDEN, axis=1), rtol=0, atol=1e-6)
    expected, expected_core = gdn_closed_form(Q_ROWS, K_ROWS, V_ROWS, Z_ROWS, A_ROWS, B_ROWS, CONV_TAPS)
    assert np.all(np.abs(got[:, 0] - expected) < 2e-4), (got[:, 0], expected)
    assert np.all(np.abs(cores - expected_core) < 2e-4), np.max(np.abs(cores - expected_core))

    # The closed form separates every plausible composition slip by far
    # more than the tolerance, so an oracle making one of them fails above.
    slips = {
        "a<->b": gdn_closed_form(Q_ROWS, K_ROWS, V_ROWS, Z_ROWS, B_ROWS, A_ROWS, CONV_TAPS),
        "q<->k": gdn_closed_form(K_ROWS, Q_ROWS, V_ROWS, Z_ROWS, A_ROWS, B_ROWS, CONV_TAPS),
        "z<->v": gdn_closed_form(Q_ROWS, K_ROWS, Z_ROWS, V_ROWS, A_ROWS, B_ROWS, CONV_TAPS),
        "taps reversed": gdn_closed_form(Q_ROWS, K_ROWS, V_ROWS, Z_ROWS, A_ROWS, B_ROWS, CONV_TAPS[::-1]),
        "heads swapped": gdn_closed_form(Q_ROWS, K_ROWS, V_ROWS, Z_ROWS, A_ROWS, B_ROWS, CONV_TAPS,
                                         out_signs=(-1.0 / 3, 1.0)),
    }
    for name, (wrong, wrong_core) in slips.items():
        assert max(np.max(np.abs(wrong - expected)), np.max(np.abs(wrong_core - expected_core))) > 1e-2, name


# ------------------------------------------------------------ MTP input order
def test_mtp_fc_input_order(orc):
    """fc over [norm_emb(embedding), norm_hid(hidden)] (decoder.rs:1027-1036).
    The embedding half of every fc row weighs 1/128 per column, the hidden
    half 3/128; norm_emb has weight 0 ((1 + w) = 1), norm_hid weight 1
    (factor 2). embedding(0) = 0.5*1 normalises to e = 0.5 / sqrt(0.25 +
    eps); prev = 2*1 normalises to 2 * 2 / sqrt(4 + eps). So every fc
    output is 64/128 * e + 64 * 3/128 * 2 * hn = 0.5 e + 3 hn (about 3.5);
    the reversed order would give 0.5 * 2 hn + 1.5 e (about 2.5)."""
    t = fixture_tensors(orc)
    one16 = lambda k: np.ones(k, np.float16).view(np.uint8)
    row = orc.q2_quantize([1.0 / 128] * HIDDEN) + orc.q2_quantize([3.0 / 128] * HIDDEN)
    t["mtp.fc"] = {"kind": "quant", "dtype": orc.Q2B64, "rows": HIDDEN, "cols": 2 * HIDDEN, "data": row * HIDDEN,
                   "s_in": one16(2 * HIDDEN), "s_out": one16(HIDDEN)}
    t["mtp.norm_hid"] = {"kind": "f32", "data": np.ones(HIDDEN, np.float32)}
    dec = decoder_with(t, interval=1)
    out = dec.mtp_fc(0, np.full(HIDDEN, 2.0, np.float32))
    e = 0.5 / math.sqrt(0.25 + EPS)
    hn = 2.0 / math.sqrt(4.0 + EPS)
    expected = 0.5 * e + 3.0 * hn
    reversed_order = 0.5 * 2.0 * hn + 1.5 * e
    assert abs(expected - reversed_order) > 0.5
    assert np.all(np.abs(out - expected) < 2e-5), (out[:4], expected)


# ------------------------------------------------------------ top-k / top-p
def truncated_law(logits, temperature, top_k, top_p):
    """Q/src/sampler.rs:85-136 stated in float64: candidates sorted by scaled
    logit descending, ties by token descending; keep the first top_k (0 =
    all); probabilities exp(l - max); keep the shortest prefix whose
    cumulative mass reaches top_p of the total. Returns the kept tokens in
    order and their cumulative mass normalised to 1."""
    scaled = [(float(l) / temperature, tok) for tok, l in enumerate(logits)]
    scaled.sort(key=lambda c: (c[0], c[1]), reverse=True)
    if top_k > 0:
        scaled = scaled[:top_k]
    mx = scaled[0][0]
    probs = [math.exp(v - mx) for v, _ in scaled]
    total = sum(probs)
    keep, acc = len(probs), 0.0
    for i, p in enumerate(probs):
        acc += p
        if acc >= top_p * total:
            keep = i + 1
            break
    probs = probs[:keep]
    tokens = [tok for _, tok in scaled[:keep]]
    cdf = np.cumsum(probs) / sum(probs)
    return tokens, cdf


def test_sampler_hand_cases(orc):
    # p = (0.4, 0.3, 0.2, 0.1) at T = 1: top_p 0.6 keeps {0, 1} (0.4 < 0.6 <= 0.7).
    logits = np.log([0.4, 0.3, 0.2, 0.1]).astype(np.float32)
    assert orc.sample_with_draw(logits, 1.0, 0, 0.6, 0.55) == 0      # 0.55 * 0.7 = 0.385 <= 0.4
    assert orc.sample_with_draw(logits, 1.0, 0, 0.6, 0.60) == 1      # 0.42 > 0.4
    assert orc.sample_with_draw(logits, 1.0, 0, 0.6, 0.999) == 1     # never token 2 or 3
    # top_p exactly on a cumulative value keeps that token (">="): 0.7 keeps {0, 1}.
    assert orc.sample_with_draw(logits, 1.0, 0, 0.7, 0.99) == 1
    # top_k 3 then top_p 1: mass 0.9, token 2 above 0.7 / 0.9.
    assert orc.sample_with_draw(logits, 1.0, 3, 1.0, 0.80) == 2
    assert orc.sample_with_draw(logits, 1.0, 3, 1.0, 0.77) == 1
    # top_k 2 on a tie for second place keeps the later token (ties: later index first).
    tie = np.array([3.0, 1.0, 1.0, 0.0], np.float32)
    assert orc.sample_with_draw(tie, 1.0, 2, 1.0, 0.999) == 2


@pytest.mark.parametrize("top_k", [2, 3, 5])
@pytest.mark.parametrize("top_p", [0.3, 0.6, 0.9])
def test_sampler_truncation_brute_force(orc, top_k, top_p):
    rng = np.random.default_rng(1000 * top_k + int(top_p * 10))
    grid = (np.arange(4000) + 0.5) / 4000.0
    for case in range(12):
        vocab = int(rng.integers(2, 9))
        logits = rng.normal(0.0, 1.5, vocab).astype(np.float32)
        if case % 3 == 0 and vocab >= 3:  # a tie across the top-k boundary
            logits[int(rng.integers(vocab))] = logits[int(rng.integers(vocab))]
        temperature = float(rng.choice([0.5, 0.8, 1.3]))
        tokens, cdf = truncated_law(logits, temperature, top_k, top_p)
        checked = 0
        for u in grid:
            if np.min(np.abs(cdf - u)) < 1e-4:  # float32 cumulative sums may land either side
                continue
            want = tokens[int(np.searchsorted(cdf, u, side="left"))]
            assert orc.sample_with_draw(logits, temperature, top_k, top_p, float(u)) == want, \
                (logits, temperature, top_k, top_p, u)
            checked += 1
        assert checked > 3900


@pytest.fixture
def tensors_crate(orc):
    return fixture_tensors(orc)


# ------------------------------------------------- MTP accept at T > 0
# Speculative rejection sampling (no crate counterpart: the crate's MTP is
# greedy), stated from its definition: draft token d of row i is accepted
# iff u * q_i(d) < p_i(d) with u the next uniform draw of the crate's Pcg32;
# on the first rejection the next token is drawn with the following uniform
# from the residual law max(p_i - q_i, 0) (normalised); when every draft is
# accepted, from the bonus row's softmax. p, q are temperature softmaxes of
# the target and draft rows. Each check below fixes a decision the
# definition determines, so a swapped ratio (q / p), a wrong residual
# (q - p), a reused or skipped draw, or the temperature left out fails.

def _softmax64(x, t):
    z = np.asarray(x, np.float64) / t
    e = np.exp(z - z.max())
    return e / e.sum()


def _draws(orc, seed, n):
    g = orc.Pcg32(seed)
    return [g.next_f32() for _ in range(n)]


@pytest.mark.parametrize("t", [0.4, 0.7, 1.3])
def test_mtp_accept_decision_is_u_q_below_p(orc, t):
    # Two tokens, one draft: the acceptance of token 0 follows u < p(0) / q(0)
    # for the first draw of every seed (cases within 1e-5 of the boundary skipped).
    target = np.array([[0.3, -0.4]], np.float32)
    draft = np.array([[0.9, -0.8]], np.float32)
    p, q = _softmax64(target[0], t), _softmax64(draft[0], t)
    ratio = p[0] / q[0]
    assert 0.2 < ratio < 0.95  # the draft over-weights token 0: a real decision
    bonus = np.zeros(2, np.float32)
    decided = 0
    for seed in range(300):
        u = _draws(orc, seed, 1)[0]
        if abs(u - ratio) < 1e-5:
            continue
        nxt, nacc = orc.mtp_accept_sample(draft, target, bonus, [0], t, orc.Pcg32(seed))
        assert nacc == (1 if u < ratio else 0), (seed, u, ratio)
        if nacc == 0:
            # residual max(p - q, 0) is all on token 1
            assert nxt == 1
        decided += 1
    assert decided > 250


def test_mtp_accept_residual_is_target_minus_draft(orc):
    # Three tokens, draft d = 2 with q(2) >> p(2): rejected for most draws.
    # p - q is positive only on token 0, so every rejection resamples token 0
    # (q - p would put the mass on token 2; an unclipped residual could give 1).
    t = 0.7
    target = np.array([[1.2, 0.1, -2.0]], np.float32)
    draft = np.array([[0.6, 0.9, 1.5]], np.float32)
    p, q = _softmax64(target[0], t), _softmax64(draft[0], t)
    assert p[0] > q[0] and p[1] < q[1] and p[2] < q[2]
    bonus = np.zeros(3, np.float32)
    rejected = 0
    for seed in range(200):
        nxt, nacc = orc.mtp_accept_sample(draft, target, bonus, [2], t, orc.Pcg32(seed))
        if nacc == 0:
            assert nxt == 0
            rejected += 1
    assert rejected > 150


def test_mtp_accept_draws_consumed_in_order(orc):
    # k = 3 drafts with identical draft and target rows accept for any draw
    # (u q < p with p = q unless u = 1, which Pcg32's f32 never returns); the
    # bonus row then puts all its mass on token 4, and the generator has
    # advanced by exactly k + 1 draws. A rejection at row 1 (draft token with
    # p = 0 there) consumes 2 + 2 draws and resamples from row 1's residual.
    t, vocab, k = 0.7, 5, 3
    rng = np.random.default_rng(4)
    rows = rng.standard_normal((k, vocab)).astype(np.float32)
    bonus = np.full(vocab, -60.0, np.float32)
    bonus[4] = 60.0
    for seed in range(20):
        g = orc.Pcg32(seed)
        nxt, nacc = orc.mtp_accept_sample(rows, rows, bonus, [1, 2, 3], t, g)
        assert (nxt, nacc) == (4, 3)
        ref = orc.Pcg32(seed)
        _ = [ref.next_f32() for _ in range(k + 1)]
        assert g.c.state == ref.c.state
    target = rows.copy()
    target[1, 3] = -np.inf  # p_1(3) = 0: draft token 3 at row 1 is always rejected
    target[1, :3] = [-60.0, -60.0, 60.0]  # the residual then sits on token 2
    draft = rows.copy()
    for seed in range(20):
        g = orc.Pcg32(seed)
        nxt, nacc = orc.mtp_accept_sample(draft, target, bonus, [1, 3, 0], t, g)
        assert (nxt, nacc) == (2, 1)
        ref = orc.Pcg32(seed)
        _ = [ref.next_f32() for _ in range(3)]  # row 0 accept, row 1 reject, row 1 residual
        assert g.c.state == ref.c.state
