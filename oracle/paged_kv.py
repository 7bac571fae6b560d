"""CPU restatement of the crate's paged mixed Q2/Q4 KV cache.

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's cpu_baseline leg
as the checker; the product path (ctox-llm_amd/) never imports it.

Follows Q/src/kv_cache.rs (Q = models/qwen38_27b):
  * QuantizedKvPage push / requantize / dequantize_token  (:170-236)
  * packed_bytes_for_values                               (:238-252)
  * PagedKvCache::new / push_internal / demote_old_pages  (:330-478)
  * projected_packed_bytes, q4/q2 token counts, page views (:500-575)
  * flattened_component: token-major pages -> head-major   (:579-605)
Blocks are quantized by the C oracle's Q4Block64 / Q2Block64 restatement
(Q/src/quant.rs:74-175). `paged_attention` is what the crate's CPU executor
computes for a full-attention layer (Q/src/decoder.rs:774-787): flatten the pages, then
grouped_query_attention (Q/src/reference.rs:420-499).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List

import numpy as np

from . import oracle as orc

Q2, Q4 = 0, 1
BLOCK_BYTES = {Q2: orc.Q2_BLOCK_BYTES, Q4: orc.Q4_BLOCK_BYTES}
Q2_CODEBOOK = np.array([-1.0, -1.0 / 3.0, 1.0 / 3.0, 1.0], np.float32)


def packed_bytes_for_values(values: int, precision: int) -> int:
    """Q/src/kv_cache.rs:238-252."""
    if values == 0 or values % orc.BLOCK_LEN:
        raise orc.OracleError(7)
    return values // orc.BLOCK_LEN * BLOCK_BYTES[precision]


def quantize_values(values, precision: int) -> bytes:
    """append_quantized (Q/src/kv_cache.rs:254-263)."""
    v = np.asarray(values, np.float32)
    q = orc.q2_quantize if precision == Q2 else orc.q4_quantize
    return b"".join(q(v[i:i + 64]) for i in range(0, v.size, 64))


def dequantize_bytes(data: bytes, precision: int) -> np.ndarray:
    """dequantize_bytes (Q/src/kv_cache.rs:265-283), vectorised over blocks.

    Q4: fp16(scale) * ((c - 7.5) / 7.5); Q2: fp16(scale) * codebook[c]
    (Q/src/quant.rs:106-111, :171-175), both in f32."""
    bb = BLOCK_BYTES[precision]
    raw = np.frombuffer(data, np.uint8).reshape(-1, bb)
    scale = raw[:, :2].copy().view(np.float16).astype(np.float32)[:, 0]
    codes = raw[:, 2:]
    if precision == Q4:
        c = np.stack([codes & 15, codes >> 4], axis=-1).reshape(-1, 64).astype(np.float32)
        n = (c - np.float32(7.5)) / np.float32(7.5)
    else:
        c = np.stack([(codes >> s) & 3 for s in (0, 2, 4, 6)], axis=-1).reshape(-1, 64)
        n = Q2_CODEBOOK[c]
    return (scale[:, None] * n).astype(np.float32).reshape(-1)


@dataclass
class Page:
    precision: int
    maximum_tokens: int
    values_per_token: int
    data: bytearray

    def token_bytes(self) -> int:
        return packed_bytes_for_values(self.values_per_token, self.precision)

    def tokens(self) -> int:
        return len(self.data) // self.token_bytes()

    def token(self, t: int) -> np.ndarray:
        tb = self.token_bytes()
        return dequantize_bytes(bytes(self.data[t * tb:(t + 1) * tb]), self.precision)

    def requantize(self, precision: int) -> None:
        """Q/src/kv_cache.rs:216-236: dequantize every token, quantize again."""
        if precision == self.precision:
            return
        out = bytearray()
        for t in range(self.tokens()):
            out += quantize_values(self.token(t), precision)
        self.precision, self.data = precision, out


class PagedKvCache:
    """Q/src/kv_cache.rs:303-605."""

    def __init__(self, maximum_tokens, component_values, page_tokens, sink_tokens, recent_tokens):
        if (maximum_tokens == 0 or page_tokens == 0 or sink_tokens > maximum_tokens
                or recent_tokens > maximum_tokens or sink_tokens % page_tokens
                or component_values == 0 or component_values % orc.BLOCK_LEN):
            raise orc.OracleError(7)
        self.maximum_tokens, self.component_values = maximum_tokens, component_values
        self.page_tokens, self.sink_tokens, self.recent_tokens = page_tokens, sink_tokens, recent_tokens
        self.n_tokens = 0
        self.pages: List[Page] = []

    def push(self, key, value, demote: bool = True):
        """push_internal (:394-429); returns (page_index, token_in_page, demoted)."""
        if self.n_tokens >= self.maximum_tokens or len(key) != self.component_values \
                or len(value) != self.component_values:
            raise orc.OracleError(7)
        if not self.pages or self.pages[-1].tokens() == self.pages[-1].maximum_tokens:
            self.pages.append(Page(Q4, min(self.page_tokens, self.maximum_tokens - self.n_tokens),
                                   2 * self.component_values, bytearray()))
        combined = np.concatenate([np.asarray(key, np.float32), np.asarray(value, np.float32)])
        # QuantizedKvPage::push (:199-206) appends in the page's precision: a
        # partial page demoted by a zero recent window takes Q2 rows.
        self.pages[-1].data += quantize_values(combined, self.pages[-1].precision)
        self.n_tokens += 1
        pi = len(self.pages) - 1
        return pi, self.pages[pi].tokens() - 1, (self.demote_old_pages() if demote else [])

    def load_pages(self, pages) -> None:
        """Replaces the contents with pages [(precision, tokens, first_token,
        bytes)] in page order, as page_views reports them (a filled cache of
        the device engine, whose page bytes are the crate's canonical ones)."""
        self.pages, self.n_tokens = [], 0
        for prec, tokens, first, data in pages:
            if first != self.n_tokens or first % self.page_tokens:
                raise orc.OracleError(7)
            p = Page(Q4 if prec else Q2, min(self.page_tokens, self.maximum_tokens - self.n_tokens),
                     2 * self.component_values, bytearray(data))
            if p.tokens() != tokens:
                raise orc.OracleError(7)
            self.pages.append(p)
            self.n_tokens += tokens

    def demote_old_pages(self) -> List[int]:
        """:463-478: a Q4 page leaves once it is past the sink and wholly older
        than the recent window."""
        recent_start = max(0, self.n_tokens - self.recent_tokens)
        demoted = []
        for i, p in enumerate(self.pages):
            start = i * self.page_tokens
            if p.precision == Q4 and start >= self.sink_tokens and start + p.tokens() <= recent_start:
                p.requantize(Q2)
                demoted.append(i)
        return demoted

    def tokens(self) -> int:
        return self.n_tokens

    def packed_bytes(self) -> int:
        return sum(len(p.data) for p in self.pages)

    def q4_tokens(self) -> int:
        return sum(p.tokens() for p in self.pages if p.precision == Q4)

    def q2_tokens(self) -> int:
        return sum(p.tokens() for p in self.pages if p.precision == Q2)

    def maximum_boundary_q4_tokens(self) -> int:
        return min(self.sink_tokens + self.recent_tokens + max(0, self.page_tokens - 1), self.maximum_tokens)

    def projected_packed_bytes(self, tokens: int) -> int:
        """:500-534."""
        if tokens > self.maximum_tokens:
            raise orc.OracleError(6)
        recent_start = max(0, tokens - self.recent_tokens)
        q2 = packed_bytes_for_values(2 * self.component_values, Q2)
        q4 = packed_bytes_for_values(2 * self.component_values, Q4)
        total = 0
        for start in range(0, tokens, self.page_tokens):
            end = min(start + self.page_tokens, tokens)
            total += (end - start) * (q4 if start < self.sink_tokens or end > recent_start else q2)
        return total

    def page_views(self):
        """(page_index, first_token, tokens, precision, bytes) per page (:558-575)."""
        return [(i, i * self.page_tokens, p.tokens(), p.precision, bytes(p.data)) for i, p in enumerate(self.pages)]

    def flattened(self, offset: int, heads: int, head_dim: int) -> np.ndarray:
        """flattened_component (:579-605): [head][token][head_dim]."""
        if heads * head_dim != self.component_values:
            raise orc.OracleError(7)
        out = np.zeros((heads, self.n_tokens, head_dim), np.float32)
        g = 0
        for p in self.pages:
            for t in range(p.tokens()):
                vals = p.token(t)[offset:offset + self.component_values].reshape(heads, head_dim)
                out[:, g, :] = vals
                g += 1
        return out.reshape(-1)

    def flattened_key(self, heads, head_dim):
        return self.flattened(0, heads, head_dim)

    def flattened_value(self, heads, head_dim):
        return self.flattened(self.component_values, heads, head_dim)


class DenseKvCache:
    """FullAttentionStorage::Dense (Q/src/decoder.rs:171-265): exact f32 K/V
    rows, chosen by FullAttentionState::new when the KV width is not a whole
    number of 64-value blocks."""

    def __init__(self, maximum_tokens, component_values):
        if maximum_tokens == 0 or component_values == 0:
            raise orc.OracleError(1)
        self.maximum_tokens, self.component_values = maximum_tokens, component_values
        self.keys, self.values = [], []

    def push(self, key, value, demote: bool = True):
        if len(self.keys) >= self.maximum_tokens or len(key) != self.component_values \
                or len(value) != self.component_values:
            raise orc.OracleError(1)
        self.keys.append(np.asarray(key, np.float32).copy())
        self.values.append(np.asarray(value, np.float32).copy())
        return len(self.keys) - 1, 0, []

    def demote_old_pages(self) -> List[int]:
        return []

    def tokens(self) -> int:
        return len(self.keys)

    def q2_tokens(self) -> int:
        return 0

    def _flat(self, rows, heads, head_dim):
        if heads * head_dim != self.component_values:
            raise orc.OracleError(1)
        a = np.stack(rows).reshape(len(rows), heads, head_dim) if rows else np.zeros((0, heads, head_dim), np.float32)
        return a.transpose(1, 0, 2).reshape(-1).copy()

    def flattened_key(self, heads, head_dim):
        return self._flat(self.keys, heads, head_dim)

    def flattened_value(self, heads, head_dim):
        return self._flat(self.values, heads, head_dim)


def paged_attention(cache: PagedKvCache, query, rows: int, query_heads: int, kv_heads: int,
                    head_dim: int) -> np.ndarray:
    """Attention of the last `rows` cached tokens' queries (query
    [rows][query_heads][head_dim]) over the cache; returns
    [rows][query_heads][head_dim]. Q/src/decoder.rs:687-800 flattens the cache
    and calls grouped_query_attention with q0 = tokens - rows (:774-787)."""
    k = cache.flattened_key(kv_heads, head_dim)
    v = cache.flattened_value(kv_heads, head_dim)
    q = np.asarray(query, np.float32).reshape(rows, query_heads, head_dim).transpose(1, 0, 2).copy()
    kvt = cache.tokens()
    return orc.grouped_query_attention(q.reshape(-1), k, v, query_heads, kv_heads, rows, kvt, head_dim,
                                       kvt - rows)
