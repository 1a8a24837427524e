"""Page pool: the on-device format of the paged KV cache.

Counterpart of kavor/engine/cache_pool.py:39-150, 292-322 for full-attention models.
One uint8 tensor [num_pools, num_blocks, page_bytes] holds every layer's pages, one
pool per attention KV slot in model order.  A page is one block of block_size tokens
of one layer, K first and V second:

    page_bytes = 2 * block_size * num_kv_heads * head_dim * itemsize   (1 MiB for Qwen3)
    k_cache[slot] = pool.view(bf16).as_strided([num_blocks, block_size, Hkv, D],
                                               [page_bytes / 2, Hkv*D, D, 1])
    v_cache[slot] = the same view offset by block_size*Hkv*D elements

so block b of a layer is one contiguous MiB of HBM, and the append and attention
kernels receive block_stride = 2*block_size*Hkv*D (cache_pool.py:311-322).  Attention
modules are found by duck typing (k_cache, v_cache, num_kv_slots; :98-101, 270-273).
Block id b names the same page in every layer, so one block table serves all layers.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class CacheLayout:
    num_pools: int        # attention KV slots in the model (one pool each)
    num_blocks: int
    block_size: int
    page_bytes: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype

    @property
    def bytes_per_block(self) -> int:
        """HBM one block id costs across all pools."""
        return self.num_pools * self.page_bytes


class CachePool:

    def __init__(self, model: torch.nn.Module, num_kv_heads: int, head_dim: int,
                 block_size: int, dtype: torch.dtype = torch.bfloat16):
        self.model = model
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.dtype = dtype
        self.slots = [(m, i) for m in model.modules()
                      if hasattr(m, "k_cache") and hasattr(m, "v_cache")
                      for i in range(m.num_kv_slots)]
        if not self.slots:
            raise ValueError("the model has no attention layer with a KV cache")
        self.layout: CacheLayout | None = None
        self.pools: torch.Tensor | None = None

    @property
    def page_bytes(self) -> int:
        return 2 * self.block_size * self.num_kv_heads * self.head_dim * self.dtype.itemsize

    def plan(self, num_blocks: int) -> CacheLayout:
        if num_blocks < 1:
            raise ValueError(f"the page pool needs at least one block, got {num_blocks}")
        return CacheLayout(len(self.slots), num_blocks, self.block_size, self.page_bytes,
                           self.num_kv_heads, self.head_dim, self.dtype)

    def blocks_for_budget(self, budget_bytes: int) -> int:
        """How many block ids fit in `budget_bytes` of device memory."""
        return max(0, budget_bytes // (len(self.slots) * self.page_bytes))

    def allocate(self, num_blocks: int, device) -> CacheLayout:
        self.release()
        layout = self.plan(num_blocks)
        self.pools = torch.empty(layout.num_pools, num_blocks, layout.page_bytes,
                                 dtype=torch.uint8, device=device)
        self._bind(layout)
        self.layout = layout
        return layout

    def release(self) -> None:
        if self.pools is None:
            return
        for module, slot in self.slots:
            module.k_cache[slot] = torch.empty(0)
            module.v_cache[slot] = torch.empty(0)
        self.pools = None
        self.layout = None

    def _bind(self, layout: CacheLayout) -> None:
        itemsize = layout.dtype.itemsize
        block_elems = layout.block_size * layout.num_kv_heads * layout.head_dim
        shape = (layout.num_blocks, layout.block_size, layout.num_kv_heads, layout.head_dim)
        strides = (layout.page_bytes // itemsize, layout.num_kv_heads * layout.head_dim,
                   layout.head_dim, 1)
        for pool, (module, slot) in enumerate(self.slots):
            flat = self.pools[pool].view(layout.dtype)
            base = flat.storage_offset()
            module.k_cache[slot] = flat.as_strided(shape, strides, base)
            module.v_cache[slot] = flat.as_strided(shape, strides, base + block_elems)

    def copy_blocks(self, src_ids: list[int], dst_ids: list[int]) -> None:
        """Whole-page copies in every pool (cache_pool.py:142-149), on the current stream."""
        if not src_ids:
            return
        if len(src_ids) != len(dst_ids):
            raise ValueError("src_ids and dst_ids differ in length")
        dev = self.pools.device
        src = torch.tensor(src_ids, dtype=torch.int64, device=dev)
        dst = torch.tensor(dst_ids, dtype=torch.int64, device=dev)
        self.pools[:, dst] = self.pools[:, src]
