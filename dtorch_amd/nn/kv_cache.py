"""KV caches for the decode loop: a padded per-sequence cache and a paged one.

The reference's Llama port keeps no cache and recomputes causal attention over the whole sequence at
every step (python/dtorch/test/modules/llama.py:126-156, with repeat_kv for GQA at :80-85).  These
classes hold the keys and values of the tokens seen so far, so that a step appends its new tokens and
attends with the split-KV decode kernels:

    cache = KVCache(batch, kv_heads, max_len, head_dim)
    out = cache.prefill(q, k, v)          # prompt: causal attention, then its K/V into the cache
    out = cache.decode(q1, k1, v1)        # one token per sequence: append, then decode attention

Prompts in one prefill call share their length; per-sequence lengths then diverge only through the
caller's own use of `lengths`.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import functional as F


class KVCache:
    """Padded cache [B, Hkv, max_len, D] plus device lengths [B] (int32)."""

    def __init__(self, batch: int, kv_heads: int, max_len: int, head_dim: int, dtype=torch.bfloat16,
                 device="cuda", scale: Optional[float] = None):
        self.k = torch.zeros(batch, kv_heads, max_len, head_dim, dtype=dtype, device=device)
        self.v = torch.zeros_like(self.k)
        self.lengths = torch.zeros(batch, dtype=torch.int32, device=device)
        self.scale = scale
        self._host_len = np.zeros(batch, dtype=np.int64)  # mirrors `lengths` for capacity checks
        self._host_stale = False  # a step was recorded under graph capture: replays outrun _host_len

    @property
    def capacity(self) -> int:
        return self.k.shape[2]

    def _span(self) -> int:
        """Cache positions the decode kernel covers.  Its split grid is sized by S_max, so in eager use the
        cache is passed as a view up to the longest sequence rather than the whole capacity (one split per
        384 tokens of S_max, empty ones included: a 32K-token cache holding 2K-token sequences would launch
        16x the workgroups).  Under graph capture, and after it until sync_lengths(), the host does not
        know the lengths the replays reach, so the whole capacity is covered."""
        if torch.cuda.is_current_stream_capturing():
            self._host_stale = True
        if self._host_stale:
            return self.capacity
        return max(int(self._host_len.max(initial=0)), 1)

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """Append [B, Hkv, n, D] keys and values after each sequence's current length."""
        n = k_new.shape[2]
        if int(self._host_len.max(initial=0)) + n > self.capacity:
            raise ValueError(f"KV cache full: {int(self._host_len.max())} + {n} tokens > capacity {self.capacity}")
        F.kv_cache_append(self.k, self.v, self.lengths, k_new, v_new)
        self._host_len += n  # only once the append was accepted

    def prefill(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """Causal attention over a prompt of equal length per sequence (the cache must be empty for the
        causal alignment to hold), then the prompt's K/V into the cache."""
        if int(self._host_len.max(initial=0)) != 0:
            raise ValueError("prefill expects an empty cache; use decode() for later tokens")
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=self.scale, enable_gqa=True)
        self.append(k, v)
        return out

    def decode(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor) -> torch.Tensor:
        """One new token per sequence: append its K/V, then attend over everything cached."""
        self.append(k_new, v_new)
        n = self._span()
        return F.decode_attention(q, self.k[:, :, :n], self.v[:, :, :n], self.lengths, scale=self.scale)[0]

    def sync_lengths(self) -> np.ndarray:
        """Refresh the host copy of the lengths from the device (one synchronising copy).

        A decode step captured in a HIP graph advances the host copy once, at capture; every replay
        advances only the device lengths.  Call this after replays and before eager use, so that the
        capacity check sees the true lengths.  The caller bounds the number of replays by
        capacity - current length: the append kernel drops tokens past the capacity (and the lengths
        saturate there), so later replays would attend over a truncated cache.
        """
        self._host_len = self.lengths.to("cpu", torch.int64).numpy().copy()
        self._host_stale = False
        return self._host_len.copy()


class PagedKVCache:
    """Paged cache: pools [num_pages, Hkv, page_size, D], a block table [B, max_pages] and lengths [B].

    Pages come from a host-side free list when a sequence's next tokens cross into a new page; the block
    table rows that change are copied to the device before the append that writes them.
    """

    def __init__(self, batch: int, kv_heads: int, num_pages: int, page_size: int, max_pages: int, head_dim: int,
                 dtype=torch.bfloat16, device="cuda", scale: Optional[float] = None):
        self.k = torch.zeros(num_pages, kv_heads, page_size, head_dim, dtype=dtype, device=device)
        self.v = torch.zeros_like(self.k)
        self.page_size = page_size
        self.scale = scale
        self._free = list(range(num_pages - 1, -1, -1))
        # unassigned slots hold -1, which names no page: the append kernel drops a token written through one
        # (a graph replay past a sequence's pages), and decode reads never reach past the length
        self._table = np.full((batch, max_pages), -1, dtype=np.int32)
        self._pages = np.zeros(batch, dtype=np.int64)  # pages assigned per sequence
        self._host_len = np.zeros(batch, dtype=np.int64)
        self.block_table = torch.from_numpy(self._table).to(device)
        self.lengths = torch.zeros(batch, dtype=torch.int32, device=device)
        self._host_stale = False  # a step was recorded under graph capture: replays outrun _host_len

    def _span_pages(self) -> int:
        """Block-table columns the decode kernel covers: the most pages any sequence holds in eager use
        (the split grid is sized by max_pages * page_size), the whole table under graph capture and after
        it until sync_lengths()."""
        if torch.cuda.is_current_stream_capturing():
            self._host_stale = True
        if self._host_stale:
            return self._table.shape[1]
        return max(int(self._pages.max(initial=0)), 1)

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        n = k_new.shape[2]
        need = (self._host_len + n + self.page_size - 1) // self.page_size
        if int(need.max(initial=0)) > self._table.shape[1]:
            raise ValueError("PagedKVCache: a sequence exceeds max_pages * page_size tokens")
        if int((need - self._pages).sum()) > len(self._free):
            raise ValueError("PagedKVCache: out of pages")
        changed = False
        for b in range(len(need)):
            while self._pages[b] < need[b]:
                self._table[b, self._pages[b]] = self._free.pop()
                self._pages[b] += 1
                changed = True
        if changed:
            self.block_table.copy_(torch.from_numpy(self._table), non_blocking=False)
        F.kv_cache_append_paged(self.k, self.v, self.block_table, self.lengths, k_new, v_new)
        self._host_len += n  # only once the append was accepted

    def prefill(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        if int(self._host_len.max(initial=0)) != 0:
            raise ValueError("prefill expects an empty cache; use decode() for later tokens")
        out = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=self.scale, enable_gqa=True)
        self.append(k, v)
        return out

    def decode(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor) -> torch.Tensor:
        self.append(k_new, v_new)
        n = self._span_pages()
        return F.decode_attention_paged(q, self.k, self.v, self.block_table[:, :n], self.lengths, scale=self.scale)[0]

    def sync_lengths(self) -> np.ndarray:
        """Refresh the host copy of the lengths from the device after HIP-graph replays.

        Replays assign no pages: the block-table slots past a sequence's assigned pages hold -1, so the
        caller bounds the replays by the tokens left on the pages already assigned.  Raises if a replay
        went past them: those tokens were dropped (no page was written) and the sequence's cache is
        incomplete.
        """
        dev = self.lengths.to("cpu", torch.int64).numpy().copy()
        if np.any(dev > self._pages * self.page_size):
            raise RuntimeError("PagedKVCache: graph replays appended past the assigned pages")
        self._host_len = dev
        self._host_stale = False
        return dev.copy()
