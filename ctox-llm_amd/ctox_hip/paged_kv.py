"""Device-resident paged mixed Q2/Q4 KV cache for one attention layer.

Host-side mirror of PagedKvCache (Q/src/kv_cache.rs:303-605) whose pages
live in HBM, as the crate's CUDA runtime keeps them: a Q4 pool and a Q2 pool
of fixed-size page slots, one descriptor {precision, physical_slot, tokens,
first_token} per logical page (CtoxPagedKvDescriptor,
q2q4_fused_matvec_sm86.cu:1614-1619), and the retention policy of
push_internal / demote_old_pages (:394-478): new tokens are packed into the
last Q4 page; a page that is past the sink and wholly older than the recent
window is rewritten into a Q2 slot and its Q4 slot is freed.

Packing, demotion and attention run on the device through the C-ABI
(ctox_hip_kv_pack_q4_device, ctox_hip_kv_demote_device,
ctox_hip_paged_gqa_device); this class only does slot bookkeeping and
descriptor uploads. Device memory comes from torch.
"""
from __future__ import annotations

import math
from typing import List, Optional

import numpy as np

from . import HipBackend, PagedGqaParams, ShapeError, MemoryBudget

Q2, Q4 = 0, 1
Q2_BLOCK_BYTES, Q4_BLOCK_BYTES = 18, 34


class DevicePagedKvCache:
    def __init__(self, backend: HipBackend, maximum_tokens: int, key_value_heads: int, head_dim: int,
                 page_tokens: int = 128, sink_tokens: int = 128, recent_tokens: int = 256,
                 q4_slots: Optional[int] = None, device: str = "cuda"):
        import torch
        cv = key_value_heads * head_dim
        # Q/src/kv_cache.rs:330-352 contract.
        if (maximum_tokens == 0 or page_tokens == 0 or sink_tokens > maximum_tokens
                or recent_tokens > maximum_tokens or sink_tokens % page_tokens or cv == 0 or cv % 64):
            raise ShapeError("invalid paged KV capacity, geometry, or retention policy")
        self.hip, self.torch = backend, torch
        self.maximum_tokens, self.page_tokens = maximum_tokens, page_tokens
        self.sink_tokens, self.recent_tokens = sink_tokens, recent_tokens
        self.kv_heads, self.head_dim, self.cv = key_value_heads, head_dim, cv
        self.q4_token_bytes = 2 * cv // 64 * Q4_BLOCK_BYTES
        self.q2_token_bytes = 2 * cv // 64 * Q2_BLOCK_BYTES
        self.q4_page_bytes = page_tokens * self.q4_token_bytes
        self.q2_page_bytes = page_tokens * self.q2_token_bytes
        pages = math.ceil(maximum_tokens / page_tokens)
        # Q4 pages at any time: the sink, the recent window and one boundary page
        # on either side (Q/src/kv_cache.rs:536-542 bounds the tokens).
        if q4_slots is None:
            q4_slots = min(pages, sink_tokens // page_tokens + math.ceil(recent_tokens / page_tokens) + 2)
        self.q4_pool = torch.zeros(q4_slots * self.q4_page_bytes, dtype=torch.uint8, device=device)
        self.q2_pool = torch.zeros(pages * self.q2_page_bytes, dtype=torch.uint8, device=device)
        self.desc = np.zeros((pages, 4), np.uint32)   # precision, slot, tokens, first_token
        self.d_desc = torch.zeros((pages, 4), dtype=torch.int32, device=device)
        self.free_q4: List[int] = list(range(q4_slots - 1, -1, -1))
        self.free_q2: List[int] = list(range(pages - 1, -1, -1))
        self.n_pages = 0
        self.n_tokens = 0

    # -- bookkeeping ----------------------------------------------------
    def _upload(self, first: int, last: int) -> None:
        if last > first:
            self.d_desc[first:last].copy_(self.torch.from_numpy(self.desc[first:last].view(np.int32)))

    def tokens(self) -> int:
        return self.n_tokens

    def q4_tokens(self) -> int:
        return int(self.desc[:self.n_pages][self.desc[:self.n_pages, 0] == Q4, 2].sum())

    def q2_tokens(self) -> int:
        return int(self.desc[:self.n_pages][self.desc[:self.n_pages, 0] == Q2, 2].sum())

    def page_views(self):
        """(page_index, first_token, tokens, precision, bytes) as Q/src/kv_cache.rs:558-575."""
        out = []
        for i in range(self.n_pages):
            prec, slot, tokens, first = (int(x) for x in self.desc[i])
            if prec == Q4:
                raw = self.q4_pool[slot * self.q4_page_bytes:slot * self.q4_page_bytes + tokens * self.q4_token_bytes]
            else:
                raw = self.q2_pool[slot * self.q2_page_bytes:slot * self.q2_page_bytes + tokens * self.q2_token_bytes]
            out.append((i, first, tokens, prec, raw.cpu().numpy().tobytes()))
        return out

    # -- push -------------------------------------------------------------
    def push(self, keys, values, demote: bool = True) -> List[int]:
        """Append rows of K and V (device float32 [n][kv_heads * head_dim]);
        returns the demoted page indices. One pack launch per page touched."""
        n = int(keys.shape[0]) if keys.dim() == 2 else 1
        keys, values = keys.reshape(n, self.cv).contiguous(), values.reshape(n, self.cv).contiguous()
        if self.n_tokens + n > self.maximum_tokens:
            raise ShapeError("paged KV append capacity or geometry differs")
        done, first_dirty, demoted = 0, self.n_pages, []
        while done < n:
            if self.n_pages == 0 or self.desc[self.n_pages - 1, 2] == self.page_tokens:
                if not self.free_q4:
                    raise MemoryBudget("no free Q4 page slot")
                self.desc[self.n_pages] = (Q4, self.free_q4.pop(), 0, self.n_pages * self.page_tokens)
                self.n_pages += 1
            page = self.n_pages - 1
            first_dirty = min(first_dirty, page)
            fill = int(self.desc[page, 2])
            take = min(n - done, self.page_tokens - fill)
            self.hip.kv_pack_q4_device(self.q4_pool.data_ptr(), keys[done].data_ptr(), values[done].data_ptr(), take,
                                       self.cv, int(self.desc[page, 1]), fill, self.q4_page_bytes)
            self.desc[page, 2] = fill + take
            done += take
            self.n_tokens += take
            # Demotion per page-sized chunk keeps at most sink + recent + 2 Q4
            # pages alive; it reaches the same pages the per-token policy does.
            if demote:
                demoted += self._demote()
        self._upload(min([first_dirty] + demoted), self.n_pages)
        return demoted

    def _demote(self) -> List[int]:
        """Q/src/kv_cache.rs:463-478."""
        recent_start = max(0, self.n_tokens - self.recent_tokens)
        out = []
        for i in range(self.n_pages):
            prec, slot, tokens, first = (int(x) for x in self.desc[i])
            if prec == Q4 and first >= self.sink_tokens and first + tokens <= recent_start:
                q2 = self.free_q2.pop()
                self.hip.kv_demote_device(self.q4_pool[slot * self.q4_page_bytes:].data_ptr(),
                                          self.q2_pool[q2 * self.q2_page_bytes:].data_ptr(), tokens,
                                          2 * self.cv // 64)
                self.free_q4.append(slot)
                self.desc[i, 0], self.desc[i, 1] = Q2, q2
                out.append(i)
        return out

    # -- attention ----------------------------------------------------------
    def params(self, query_heads: int) -> PagedGqaParams:
        return PagedGqaParams(query_heads, self.kv_heads, self.head_dim, self.n_tokens, self.page_tokens,
                              max(1, self.n_pages), 2 * self.cv, self.q2_token_bytes, self.q4_token_bytes,
                              self.q2_page_bytes, self.q4_page_bytes, 1.0 / math.sqrt(self.head_dim))

    def attention(self, query, rows: int, query_heads: int, out=None):
        """Attention of the last `rows` cached tokens' queries (device
        [rows][query_heads][head_dim]); returns the same shape."""
        if out is None:
            out = self.torch.empty((rows, query_heads, self.head_dim), dtype=self.torch.float32,
                                   device=query.device)
        self.hip.paged_gqa_device(query.data_ptr(), self.q2_pool.data_ptr(), self.q4_pool.data_ptr(),
                                  self.d_desc.data_ptr(), self.params(query_heads), rows, out.data_ptr())
        return out
