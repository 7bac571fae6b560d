"""GPU parity of the paged mixed Q2/Q4 KV cache and split-KV attention.

* Packing and demotion are byte-exact against the oracle's restatement of
  Q/src/kv_cache.rs (every page's bytes compared after every push batch,
  Q4 and demoted Q2 pages alike), including all-zero, constant, tiny and
  rounding-tie blocks.
* Attention output against the oracle (flattened pages + the
  grouped_query_attention restatement, Q/src/reference.rs:420-499) within
  rtol 1e-3 plus an absolute 1e-4 x max|out| floor (fp32 MFMA sums in a
  different order than the sequential oracle).
"""
import sys

import numpy as np
import pytest
import torch

from oracle import paged_kv as pk

pytestmark = pytest.mark.gpu

QH, KVH, HD = 24, 4, 256


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make_caches(hip, maximum, page, sink, recent):
    from ctox_hip.paged_kv import DevicePagedKvCache
    dev = DevicePagedKvCache(hip, maximum, KVH, HD, page, sink, recent)
    ref = pk.PagedKvCache(maximum, KVH * HD, page, sink, recent)
    return dev, ref


def push_both(dev, ref, keys, values):
    demoted_ref = []
    for k, v in zip(keys, values):
        demoted_ref += ref.push(k, v)[2]
    demoted = dev.push(torch.from_numpy(keys).cuda(), torch.from_numpy(values).cuda())
    torch.cuda.synchronize()
    return demoted, demoted_ref


def check_pages(dev, ref):
    dv, rv = dev.page_views(), ref.page_views()
    assert len(dv) == len(rv)
    for a, b in zip(dv, rv):
        assert a[:4] == b[:4], (a[:4], b[:4])
        if a[4] != b[4]:
            x, y = np.frombuffer(a[4], np.uint8), np.frombuffer(b[4], np.uint8)
            bad = np.nonzero(x != y)[0]
            raise AssertionError(f"page {a[0]} differs at {bad[:8]} of {x.size}: {x[bad[:8]]} vs {y[bad[:8]]}")


def special_rows(rng, n):
    cv = KVH * HD
    k = (rng.standard_normal((n, cv)) * 2).astype(np.float32)
    v = (rng.standard_normal((n, cv)) * 2).astype(np.float32)
    k[0, :64] = 0.0                                   # zero block
    k[0, 64:128] = 3.25                               # constant block
    v[0, :64] = 1e-30                                 # fp16 scale underflows to zero
    m = np.float32(4.0)                               # rounding ties: n * 7.5 + 7.5 = x.5
    k[1, :64] = m * ((np.arange(64) % 15 + 0.5 - 7.5) / 7.5).astype(np.float32)
    k[1, 0] = m
    v[1, :64] = np.float32(70000.0) * rng.standard_normal(64).astype(np.float32) / 10
    return k, v


def test_pack_and_demote_match_oracle(hip):
    say("case paged pack/demote page=16 sink=32 recent=64")
    rng = np.random.default_rng(1)
    dev, ref = make_caches(hip, 512, 16, 32, 64)
    total = 0
    for n in [1, 5, 37, 2, 100, 16, 3, 64, 1, 1]:
        k, v = special_rows(rng, n) if n >= 2 else (rng.standard_normal((n, KVH * HD)).astype(np.float32),
                                                     rng.standard_normal((n, KVH * HD)).astype(np.float32))
        demoted, demoted_ref = push_both(dev, ref, k, v)
        total += n
        assert sorted(demoted) == sorted(demoted_ref)
        check_pages(dev, ref)
    assert dev.tokens() == ref.tokens() == total
    assert dev.q2_tokens() == ref.q2_tokens() > 0 and dev.q4_tokens() == ref.q4_tokens()


def attention_case(hip, tokens, rows, page, sink, recent, seed):
    rng = np.random.default_rng(seed)
    dev, ref = make_caches(hip, max(tokens + 8, sink + recent), page, sink, recent)
    cv = KVH * HD
    k = (rng.standard_normal((tokens, cv)) * 1.5).astype(np.float32)
    v = rng.standard_normal((tokens, cv)).astype(np.float32)
    push_both(dev, ref, k, v)
    q = (rng.standard_normal((rows, QH, HD)) * 1.5).astype(np.float32)
    dq = torch.from_numpy(q).cuda()
    out = dev.attention(dq, rows, QH)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = pk.paged_attention(ref, q, rows, QH, KVH, HD).reshape(rows, QH, HD)
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-4 * float(np.abs(want).max()))
    return dev, ref


@pytest.mark.parametrize("tokens,rows,page,sink,recent", [
    (1, 1, 16, 0, 16), (7, 5, 16, 0, 16), (16, 1, 16, 16, 16), (37, 3, 16, 16, 16),
    (300, 5, 16, 32, 64), (300, 1, 16, 32, 64), (1000, 2, 128, 128, 256), (4096, 5, 128, 128, 256),
    (300, 5, 24, 48, 64), (100, 3, 8, 0, 16),   # pages that split 16-token tiles
    (32768, 1, 16, 128, 256), (32768, 5, 16, 128, 256),   # config 5: 32k context, page 16
])
@pytest.mark.timeout(600)
def test_paged_attention_matches_oracle(hip, tokens, rows, page, sink, recent):
    say(f"case paged attention tokens={tokens} rows={rows} page={page}")
    attention_case(hip, tokens, rows, page, sink, recent, seed=tokens * 7 + rows)


@pytest.mark.parametrize("page", [16, 24])
def test_paged_attention_value_scale_range(hip, page):
    say(f"case paged attention value scales 1e-3..1e3 page={page}")
    # Value blocks whose magnitudes differ by six orders across tokens: the
    # page-aligned kernel rescales its f16 probability operands per tile.
    rng = np.random.default_rng(11)
    tokens, rows = 700, 5
    dev, ref = make_caches(hip, 720, page, 48, 96)
    cv = KVH * HD
    k = rng.standard_normal((tokens, cv)).astype(np.float32)
    mag = 10.0 ** rng.uniform(-3, 3, (tokens, cv // 64))
    v = (rng.standard_normal((tokens, cv)) * np.repeat(mag, 64, axis=1)).astype(np.float32)
    push_both(dev, ref, k, v)
    q = rng.standard_normal((rows, QH, HD)).astype(np.float32)
    out = dev.attention(torch.from_numpy(q).cuda(), rows, QH)
    torch.cuda.synchronize()
    want = pk.paged_attention(ref, q, rows, QH, KVH, HD).reshape(rows, QH, HD)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-3, atol=1e-4 * float(np.abs(want).max()))


def test_paged_attention_peaked_scores(hip):
    say("case paged attention peaked")
    # Large logits make the softmax nearly one-hot; the online max must track it.
    rng = np.random.default_rng(9)
    dev, ref = make_caches(hip, 520, 16, 32, 64)
    k = (rng.standard_normal((500, KVH * HD)) * 6).astype(np.float32)
    v = rng.standard_normal((500, KVH * HD)).astype(np.float32)
    push_both(dev, ref, k, v)
    q = (rng.standard_normal((4, QH, HD)) * 6).astype(np.float32)
    out = dev.attention(torch.from_numpy(q).cuda(), 4, QH)
    torch.cuda.synchronize()
    want = pk.paged_attention(ref, q, 4, QH, KVH, HD).reshape(4, QH, HD)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-3, atol=1e-4 * float(np.abs(want).max()))


def test_paged_attention_errors(hip):
    import ctox_hip
    from ctox_hip.paged_kv import DevicePagedKvCache
    dev = DevicePagedKvCache(hip, 64, KVH, HD, 16, 16, 16)
    dev.push(torch.zeros(8, KVH * HD, device="cuda"), torch.zeros(8, KVH * HD, device="cuda"))
    q = torch.zeros(9, QH, HD, device="cuda")
    with pytest.raises(ctox_hip.ShapeError):
        dev.attention(q, 9, QH)                      # more rows than cached tokens
    with pytest.raises(ctox_hip.UnsupportedOperation):
        dev.attention(q, 6, QH + 12)                 # 9 heads per kv head x 6 rows > 32
    p = dev.params(QH)
    p.head_dim = 128
    with pytest.raises(ctox_hip.UnsupportedOperation):
        hip.paged_gqa_device(q.data_ptr(), dev.q2_pool.data_ptr(), dev.q4_pool.data_ptr(), dev.d_desc.data_ptr(), p, 1,
                             q.data_ptr())


@pytest.mark.parametrize("rows,pos0,slot_of", [(1, 4093, [3]), (5, 30, [1, 1, 0, 0, 0]), (8, 70000, [2] * 8)])
def test_attn_prep_fused(hip, rows, pos0, slot_of):
    """Fused q/k norm + partial RoPE + Q4 append against the oracle: q within
    the RoPE/norm tolerances of test_gpu_layer_ops; V blocks byte-exact with
    Q4Block64::quantize of the raw rows; K blocks byte-exact with the
    quantize of the oracle's normed, rotated keys except where that value lies
    within 1e-5 (relative) of a code boundary."""
    from oracle import oracle as orc
    say(f"case attn prep rows={rows} pos0={pos0}")
    qh, kvh, hd, rd, theta, eps = 24, 4, 256, 64, 1e7, 1e-6
    rng = np.random.default_rng(rows * 31 + pos0)
    rq = 2 * (qh + kvh) * hd + 8                       # q|gate per head, k, v, slack
    proj = (rng.standard_normal((rows, rq)) * 1.7).astype(np.float32)
    qn = (rng.standard_normal(hd) * 0.3).astype(np.float32)
    kn = (rng.standard_normal(hd) * 0.3).astype(np.float32)
    page_tokens = 16
    tb = 2 * kvh * hd // 64 * 34
    page_bytes = page_tokens * tb
    pages = torch.zeros(4 * page_bytes, dtype=torch.uint8, device="cuda")
    pos_in = [(7 + t) % page_tokens for t in range(rows)]
    pos_in = [pos_in[t] if slot_of.count(slot_of[t]) == 1 else t % page_tokens for t in range(rows)]
    q_out = torch.empty(rows * qh * hd, dtype=torch.float32, device="cuda")
    dproj, dqn, dkn = (torch.from_numpy(x).cuda() for x in (proj, qn, kn))
    hip.attn_prep_device(dproj.data_ptr(), rq, dqn.data_ptr(), dkn.data_ptr(), rows, qh, kvh, hd, rd, pos0, theta, eps,
                         pages.data_ptr(), page_bytes, slot_of, pos_in, q_out.data_ptr())
    torch.cuda.synchronize()
    got_q = q_out.cpu().numpy().reshape(rows, qh, hd)
    raw = pages.cpu().numpy()
    for t in range(rows):
        q = np.stack([proj[t, h * 2 * hd:h * 2 * hd + hd] for h in range(qh)])
        k = proj[t, 2 * qh * hd:2 * qh * hd + kvh * hd].reshape(kvh, hd)
        v = proj[t, 2 * qh * hd + kvh * hd:2 * (qh + kvh) * hd].reshape(kvh, hd)
        nq = orc.rms_norm_1p_weight(q.reshape(-1), qh, hd, qn, eps).reshape(qh, hd).copy()
        nk = orc.rms_norm_1p_weight(k.reshape(-1), kvh, hd, kn, eps).reshape(kvh, hd).copy()
        fq, fk = nq.reshape(-1).copy(), nk.reshape(-1).copy()
        orc.apply_partial_rope(fq, fk, qh, kvh, hd, rd, pos0 + t, theta)
        tol = 4 * float(np.spacing(np.float32(max(pos0 + t, 1)))) * 2 * 4.5 * np.abs(nq).max() + 1e-5
        np.testing.assert_allclose(got_q[t], fq.reshape(qh, hd), rtol=1e-5, atol=tol)
        off = slot_of[t] * page_bytes + pos_in[t] * tb
        tok = raw[off:off + tb].tobytes()
        assert tok[kvh * 4 * 34:] == pk.quantize_values(v.reshape(-1), pk.Q4)
        want_k = pk.quantize_values(fk, pk.Q4)
        if tok[:kvh * 4 * 34] != want_k:
            fkb = fk.reshape(-1, 64)
            for b in range(fkb.shape[0]):
                g, w = tok[b * 34:(b + 1) * 34], want_k[b * 34:(b + 1) * 34]
                if g == w:
                    continue
                m = np.abs(fkb[b]).max()
                sel = np.clip(fkb[b] / m, -1, 1) * 7.5 + 7.5
                near = np.abs(sel - np.floor(sel) - 0.5) < 1e-5 * 16
                gc = np.array([(g[2 + i // 2] >> (4 * (i % 2))) & 15 for i in range(64)])
                wc = np.array([(w[2 + i // 2] >> (4 * (i % 2))) & 15 for i in range(64)])
                assert np.all((gc == wc) | near), f"row {t} K block {b} codes differ away from a rounding boundary"
