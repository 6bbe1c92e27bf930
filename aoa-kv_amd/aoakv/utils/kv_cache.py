"""Paged KV pool and per-sequence page list.

Mirrors the reference's KvPool / KvCache (kernels/aoa_kv/quest/utils/
kv_cache.py:7-133): one device buffer per layer stack, pages handed out from
a free list, and a per-sequence list of page indices.
"""
from __future__ import annotations

import random
from typing import List, Optional

import torch

from .utils import TensorLayout


class KvPool:
    """Device buffer [num_layers, capacity, 2, page, H, D] (NHD) or
    [num_layers, capacity, 2, H, page, D] (HND) plus a free list."""

    def __init__(self, num_layers: int, num_heads: int, head_dim: int, capacity: int,
                 block_len: int, dtype: torch.dtype, device, layout: int = TensorLayout.NHD,
                 shuffle_seed: Optional[int] = None):
        self._layout = layout
        if layout == TensorLayout.NHD:
            shape = (num_layers, capacity, 2, block_len, num_heads, head_dim)
        else:
            shape = (num_layers, capacity, 2, num_heads, block_len, head_dim)
        self._buf = torch.empty(shape, dtype=dtype, device=device)
        # free list; handed out lowest-first (or in a seeded random order, to
        # exercise non-identity page tables)
        free = list(range(capacity))
        if shuffle_seed is not None:
            random.Random(shuffle_seed).shuffle(free)
        self._free: List[int] = free[::-1]

    @property
    def layout(self):
        return self._layout

    @property
    def buf(self):
        return self._buf

    @property
    def num_layers(self):
        return self._buf.shape[0]

    @property
    def block_len(self):
        return self._buf.shape[3] if self._layout == TensorLayout.NHD else self._buf.shape[4]

    @property
    def num_free_blocks(self):
        return len(self._free)

    @property
    def capacity(self):
        return self._buf.shape[1]

    def alloc_block(self) -> int:
        if not self._free:
            raise RuntimeError("KvPool exhausted")
        return self._free.pop()

    def free_block(self, idx: int):
        assert 0 <= idx < self.capacity
        assert idx not in self._free
        self._free.append(idx)


class KvCache:
    """Page list of one sequence (reference kv_cache.py:77-133)."""

    def __init__(self, num_layers, num_heads, head_dim, max_seq_len: int, page_size,
                 dtype: torch.dtype, device, layout: int = TensorLayout.NHD,
                 shuffle_seed: Optional[int] = None):
        if max_seq_len <= 0:
            raise ValueError("max_seq_len must be positive")
        self._pool = KvPool(num_layers, num_heads, head_dim,
                            (max_seq_len + page_size - 1) // page_size, page_size, dtype,
                            device, layout, shuffle_seed)
        self._indicies: List[int] = []
        self._seqlen = 0

    @property
    def pool(self) -> KvPool:
        return self._pool

    @property
    def seqlen(self) -> int:
        return self._seqlen

    @property
    def last_page_len(self) -> int:
        return (self.seqlen - 1) % self._pool.block_len + 1

    @property
    def indicies(self) -> List[int]:
        return self._indicies

    def buf_layer(self, layer_idx: int):
        assert layer_idx < self.pool.num_layers
        return self._pool.buf[layer_idx]

    def append_seq(self, seq_len: int) -> int:
        """Reserve space for tokens; return the number of new pages."""
        if seq_len <= 0:
            return 0
        new = 0
        for _ in range(seq_len):
            if self._seqlen == 0 or self.last_page_len == self._pool.block_len:
                self._indicies.append(self._pool.alloc_block())
                new += 1
            self._seqlen += 1
        return new

    def release(self):
        self._seqlen = 0
        for idx in self._indicies:
            self._pool.free_block(idx)
        self._indicies.clear()
