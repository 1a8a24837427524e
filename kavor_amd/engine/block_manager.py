"""Page accounting with prefix caching for the paged KV cache.

Counterpart of kavor/engine/block_manager.py (full-attention part; the linear-attention
state bundles, :29-41 and :270-296, belong to Qwen3.5-style models and are not part of
the paged KV path).  The observable behaviour follows the reference:

- pages come from a FIFO free list; a freed page keeps its content hash so a later
  request with the same prefix can take it back (block_manager.py:72-92);
- a full block's key is a chain hash of its parent's key and its token ids
  (:61-67); a lookup hit is only trusted after comparing the stored token ids
  (:105-107), so a hash collision cannot alias two different prefixes;
- the last block of a prompt is never taken from the cache, so prefill always has at
  least one token to compute (:99, range(num_blocks - 1));
- pages shared with running sequences are reference counted (:152-160);
- a page that is handed out again drops its stale hash entry (:76-77).

The hash itself differs from the reference (BLAKE2b-128 over the parent key and the
little-endian int64 token ids, instead of SHA-256 over a pickle): keys never leave the
process, so only the chaining and the collision check matter.
"""

from __future__ import annotations

import hashlib
from collections import deque

import numpy as np

from kavor_amd.engine.sequence import Sequence

_ROOT_KEY = b"\x00" * 16


class Block:
    """One physical page: reference count plus the key of the full block it holds."""

    __slots__ = ("block_id", "ref_count", "hash", "token_ids")

    def __init__(self, block_id: int):
        self.block_id = block_id
        self.ref_count = 0
        self.hash: bytes | None = None
        self.token_ids: list[int] = []

    def update(self, key: bytes, token_ids: list[int]) -> None:
        self.hash = key
        self.token_ids = token_ids

    def reset(self) -> None:
        self.ref_count = 1
        self.hash = None
        self.token_ids = []


class BlockManager:

    def __init__(self, num_blocks: int, block_size: int):
        if num_blocks < 1:
            raise ValueError(f"the page pool needs at least one block, got {num_blocks}")
        if block_size < 2:
            # may_append_block keys on len % block_size == 1
            raise ValueError(f"block_size must be >= 2, got {block_size}")
        self.block_size = block_size
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.hash_to_block_id: dict[bytes, int] = {}
        self.free_block_ids: deque[int] = deque(range(num_blocks))
        self.used_block_ids: set[int] = set()
        # prefix-cache counters, accumulated once per prefill allocation
        self.prefix_cache_hit_tokens = 0
        self.prefix_cache_prompt_tokens = 0

    @staticmethod
    def hash_block_tokens(parent: bytes | None, token_ids: list[int]) -> bytes:
        """Key of a full block given its parent's key (None for the first block)."""
        h = hashlib.blake2b(digest_size=16)
        h.update(parent if parent is not None else _ROOT_KEY)
        h.update(np.asarray(token_ids, dtype="<i8").tobytes())
        return h.digest()

    # ------------------------------------------------------------------ pages

    def allocate_block(self) -> int:
        block_id = self.free_block_ids.popleft()
        block = self.blocks[block_id]
        assert block.ref_count == 0, f"free block {block_id} still referenced"
        if block.hash is not None and self.hash_to_block_id.get(block.hash) == block_id:
            del self.hash_to_block_id[block.hash]
        block.reset()
        self.used_block_ids.add(block_id)
        return block_id

    def deallocate_block(self, block_id: int) -> None:
        assert self.blocks[block_id].ref_count == 0, f"block {block_id} still referenced"
        self.used_block_ids.remove(block_id)
        self.free_block_ids.append(block_id)

    def _take_cached(self, block_id: int) -> None:
        block = self.blocks[block_id]
        if block_id in self.used_block_ids:
            block.ref_count += 1
        else:
            block.ref_count = 1
            self.free_block_ids.remove(block_id)
            self.used_block_ids.add(block_id)

    # ------------------------------------------------------------------ prefill

    def _cached_prefix(self, seq: Sequence):
        """Yields (block index, block id) of the leading blocks found in the cache."""
        key = None
        for i in range(seq.num_blocks - 1):
            token_ids = seq.block(i)
            key = self.hash_block_tokens(key, token_ids)
            block_id = self.hash_to_block_id.get(key)
            if block_id is None or self.blocks[block_id].token_ids != token_ids:
                return
            yield i, block_id

    def can_allocate_prefill(self, seq: Sequence) -> int:
        """Number of leading blocks a prefill of `seq` can take from the cache, or -1
        if the free list cannot supply the rest."""
        num_cached = 0
        num_needed = seq.num_blocks
        for _, block_id in self._cached_prefix(seq):
            num_cached += 1
            if block_id in self.used_block_ids:
                num_needed -= 1
        if len(self.free_block_ids) < num_needed:
            return -1
        return num_cached

    def allocate_prefill(self, seq: Sequence, num_cached_blocks: int) -> None:
        assert not seq.block_table, "sequence already owns pages"
        taken = 0
        for _, block_id in self._cached_prefix(seq):
            if taken == num_cached_blocks:
                break
            self._take_cached(block_id)
            seq.block_table.append(block_id)
            taken += 1
        assert taken == num_cached_blocks, "cache changed between can_allocate_prefill and allocate_prefill"
        for _ in range(num_cached_blocks, seq.num_blocks):
            seq.block_table.append(self.allocate_block())
        seq.num_cached_tokens = num_cached_blocks * self.block_size
        self.prefix_cache_hit_tokens += seq.num_cached_tokens
        self.prefix_cache_prompt_tokens += seq.num_tokens

    def deallocate(self, seq: Sequence) -> None:
        # tail first, so that the prefix pages stay in the free list longest
        for block_id in reversed(seq.block_table):
            block = self.blocks[block_id]
            block.ref_count -= 1
            if block.ref_count == 0:
                self.deallocate_block(block_id)
        seq.num_cached_tokens = 0
        seq.block_table.clear()

    # ------------------------------------------------------------------ decode

    def can_append_block(self, seq: Sequence) -> bool:
        return len(self.free_block_ids) >= (len(seq) % self.block_size == 1)

    def may_append_block(self, seq: Sequence) -> None:
        if len(seq) % self.block_size == 1:
            seq.block_table.append(self.allocate_block())

    # ------------------------------------------------------------------ after a step

    def hash_blocks(self, seq: Sequence) -> None:
        """Keys the blocks that the current step fills completely."""
        start = seq.num_cached_tokens // self.block_size
        end = (seq.num_cached_tokens + seq.num_scheduled_tokens) // self.block_size
        if start == end:
            return
        key = self.blocks[seq.block_table[start - 1]].hash if start > 0 else None
        for i in range(start, end):
            block = self.blocks[seq.block_table[i]]
            token_ids = seq.block(i)
            key = self.hash_block_tokens(key, token_ids)
            block.update(key, token_ids)
            self.hash_to_block_id[key] = block.block_id
