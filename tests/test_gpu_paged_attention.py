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
])
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
