"""Pins the paged KV oracle (oracle/paged_kv.py) on the CPU.

* The crate's own tests of Q/src/kv_cache.rs (:639-676, :717-744, :746-758)
  restated with the same inputs and expected values.
* Block dequantization against the C oracle's per-element Q4/Q2 values.
* The page demotion identity the device kernel relies on: requantizing a
  dequantized Q4 block to Q2 (Q/src/kv_cache.rs:216-236) equals mapping each
  code c <= 2 -> 0, <= 7 -> 1, <= 12 -> 2, else 3 with the fp16 scale kept
  (all-zero block when the scale is zero), over random, tiny, subnormal-scale,
  constant and zero blocks.
* paged_attention against a float64 softmax attention written out directly.
"""
import numpy as np
import pytest

from oracle import paged_kv as pk
from oracle import oracle as orc_mod


def test_demotes_only_pages_outside_sink_and_recent_windows(orc):
    # Q/src/kv_cache.rs:639-676
    cache = pk.PagedKvCache(16, 64, 4, 4, 4)
    for token in range(16):
        _, _, demoted = cache.push(np.full(64, token, np.float32), np.full(64, -token, np.float32))
        if token == 11:
            assert demoted == [1]
    assert cache.tokens() == 16
    assert cache.q4_tokens() == 8
    assert cache.maximum_boundary_q4_tokens() == 11
    assert cache.packed_bytes() == 8 * 2 * 34 + 8 * 2 * 18
    assert cache.projected_packed_bytes(16) == cache.packed_bytes()
    views = cache.page_views()
    assert len(views) == 4
    assert views[0][1] == 0 and views[1][1] == 4
    assert views[1][3] == pk.Q2
    assert views[3][2] == 4 and len(views[3][4]) == 4 * 2 * 34
    key, value = cache.flattened_key(1, 64), cache.flattened_value(1, 64)
    assert key.size == 16 * 64 and value.size == 16 * 64
    assert np.isfinite(key).all() and np.isfinite(value).all()


def test_flattens_token_major_pages_into_head_major(orc):
    # Q/src/kv_cache.rs:717-744
    cache = pk.PagedKvCache(4, 128, 2, 0, 4)
    for token in range(4):
        key = np.zeros(128, np.float32)
        value = np.zeros(128, np.float32)
        key[:64], key[64:] = token + 1, token + 11
        value[:64], value[64:] = -(token + 1), -(token + 11)
        cache.push(key, value)
    key, value = cache.flattened_key(2, 64), cache.flattened_value(2, 64)
    for head in range(2):
        for token in range(4):
            expected = token + 1 + head * 10
            s = (head * 4 + token) * 64
            assert np.all(np.abs(key[s:s + 64] - expected) < 1e-3)
            assert np.all(np.abs(value[s:s + 64] + expected) < 1e-3)


def test_qwen_128k_projected_bytes_match_release_formula(orc):
    # Q/src/kv_cache.rs:746-758 (4 kv heads x 256, qwen_default policy)
    cv = 4 * 256
    cache = pk.PagedKvCache(131072, cv, 128, 128, 256)
    per_layer_q2 = 131072 * cv * 2 // 64 * 18
    q4_delta = 384 * cv * 2 // 64 * (34 - 18)
    assert cache.projected_packed_bytes(131072) == per_layer_q2 + q4_delta


def test_dequantize_matches_c_oracle(orc):
    rng = np.random.default_rng(5)
    vals = (rng.standard_normal(64 * 6) * rng.uniform(0.01, 50)).astype(np.float32)
    for prec, qfun, vfun in ((pk.Q4, orc.q4_quantize, orc.q4_value), (pk.Q2, orc.q2_quantize, orc.q2_value)):
        data = pk.quantize_values(vals, prec)
        got = pk.dequantize_bytes(data, prec)
        for b in range(6):
            blk = data[b * pk.BLOCK_BYTES[prec]:(b + 1) * pk.BLOCK_BYTES[prec]]
            ref = np.array([vfun(blk, i) for i in range(64)], np.float32)
            assert np.array_equal(got[b * 64:(b + 1) * 64].view(np.uint32), ref.view(np.uint32))


def code_map_demote(q4: bytes) -> bytes:
    """The device demotion rule, restated for the CPU check."""
    m = np.array([0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 3, 3, 3], np.uint8)
    raw = np.frombuffer(q4, np.uint8).reshape(-1, 34)
    out = np.zeros((raw.shape[0], 18), np.uint8)
    for i, blk in enumerate(raw):
        if (int(blk[0]) | (int(blk[1]) << 8)) & 0x7FFF == 0:
            continue
        out[i, :2] = blk[:2]
        codes = np.stack([blk[2:] & 15, blk[2:] >> 4], -1).reshape(64)
        q2 = m[codes].reshape(16, 4)
        out[i, 2:] = q2[:, 0] | (q2[:, 1] << 2) | (q2[:, 2] << 4) | (q2[:, 3] << 6)
    return out.tobytes()


def test_demotion_code_map_equals_requantize(orc):
    rng = np.random.default_rng(11)
    blocks = []
    for i in range(400):
        mag = 10.0 ** rng.uniform(-9, 4)  # down to fp16-subnormal and zero scales
        blocks.append((rng.standard_normal(64) * mag).astype(np.float32))
    blocks.append(np.zeros(64, np.float32))
    blocks.append(np.full(64, 3.25, np.float32))
    blocks.append(np.full(64, -1e-30, np.float32))
    blocks.append(np.linspace(-1, 1, 64).astype(np.float32))
    for v in blocks:
        q4 = pk.quantize_values(v, pk.Q4)
        requant = pk.quantize_values(pk.dequantize_bytes(q4, pk.Q4), pk.Q2)
        assert code_map_demote(q4) == requant


def attention_f64(q, k, v, rows, qh, kvh, hd, tokens):
    g = qh // kvh
    k = k.reshape(kvh, tokens, hd).astype(np.float64)
    v = v.reshape(kvh, tokens, hd).astype(np.float64)
    out = np.zeros((rows, qh, hd))
    for t in range(rows):
        n = tokens - rows + t + 1
        for h in range(qh):
            s = k[h // g, :n] @ q[t, h].astype(np.float64) / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[t, h] = p @ v[h // g, :n] / p.sum()
    return out


def test_paged_attention_oracle_matches_f64(orc):
    rng = np.random.default_rng(3)
    qh, kvh, hd, rows = 6, 2, 64, 3
    cache = pk.PagedKvCache(64, kvh * hd, 8, 8, 16)
    for _ in range(40):
        cache.push(rng.standard_normal(kvh * hd).astype(np.float32), rng.standard_normal(kvh * hd).astype(np.float32))
    assert cache.q2_tokens() > 0 and cache.q4_tokens() > 0
    q = rng.standard_normal((rows, qh, hd)).astype(np.float32)
    got = pk.paged_attention(cache, q, rows, qh, kvh, hd).reshape(rows, qh, hd)
    ref = attention_f64(q, cache.flattened_key(kvh, hd), cache.flattened_value(kvh, hd), rows, qh, kvh, hd, 40)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


def test_paged_cache_contract_errors(orc):
    with pytest.raises(orc_mod.OracleError):
        pk.PagedKvCache(16, 64, 4, 3, 4)   # sink not a page multiple
    with pytest.raises(orc_mod.OracleError):
        pk.PagedKvCache(16, 60, 4, 4, 4)   # width not a block multiple
    cache = pk.PagedKvCache(1, 64, 4, 0, 1)
    cache.push(np.zeros(64), np.zeros(64))
    with pytest.raises(orc_mod.OracleError):
        cache.push(np.zeros(64), np.zeros(64))


def test_zero_recent_window_appends_in_page_precision(orc):
    """Q/src/kv_cache.rs:199-206, 463-478: with recent 0 the page being filled
    is demoted after each push and later tokens are appended to it as Q2."""
    from oracle import paged_kv as pk
    c = pk.PagedKvCache(64, 64, 16, 0, 0)
    rng = np.random.default_rng(0)
    rows = rng.standard_normal((3, 2, 64)).astype(np.float32)
    for k, v in rows:
        c.push(k, v)
    assert c.q2_tokens() == 3 and c.q4_tokens() == 0
    want = np.concatenate([pk.dequantize_bytes(pk.quantize_values(np.concatenate([k, v]), pk.Q2), pk.Q2)
                           for k, v in rows[1:]])
    got = np.concatenate([c.pages[0].token(t) for t in (1, 2)])
    np.testing.assert_array_equal(got, want)
