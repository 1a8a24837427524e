"""Seeded input builders shared by the CPU and GPU tests (all tensors start on the CPU)."""

from __future__ import annotations

import math

import torch

from oracle import kvpath_oracle as ref

TOL = dict(atol=2e-2, rtol=1e-2)  # bf16 attention output vs the fp32 oracle


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def randn_bf16(shape, g: torch.Generator, scale: float = 1.0) -> torch.Tensor:
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def interleaved_pool(num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int,
                     g: torch.Generator) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Kavor's page layout (cache_pool.py:311-322): one uint8 [num_blocks, page_bytes] pool
    per layer, K in the first half of each page and V in the second.  Filled with random
    bf16 so untouched slots are checkable.  Returns (pool, k_cache, v_cache)."""
    page_elems = 2 * block_size * num_kv_heads * head_dim
    flat = randn_bf16((num_blocks, page_elems), g)
    pool = flat.view(torch.uint8).reshape(num_blocks, page_elems * 2)
    k_cache, v_cache = ref.page_views(pool, block_size, num_kv_heads, head_dim)
    return pool, k_cache, v_cache


def contiguous_caches(num_blocks, block_size, num_kv_heads, head_dim, g):
    shape = (num_blocks, block_size, num_kv_heads, head_dim)
    return randn_bf16(shape, g), randn_bf16(shape, g)


def qkv_views(num_tokens: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
              g: torch.Generator) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """q, k, v as in Qwen3 (kavor/models/qwen3.py:80-88): q and k fresh contiguous tensors
    (q/k RMSNorm outputs), v a strided view of the fused qkv projection output."""
    width = (num_q_heads + 2 * num_kv_heads) * head_dim
    qkv = randn_bf16((num_tokens, width), g)
    q = randn_bf16((num_tokens, num_q_heads, head_dim), g)
    k = randn_bf16((num_tokens, num_kv_heads, head_dim), g)
    v = qkv[:, (num_q_heads + num_kv_heads) * head_dim:].view(num_tokens, num_kv_heads, head_dim)
    return q, k, v


def random_block_tables(context_lens: list[int], block_size: int, num_blocks: int,
                        g: torch.Generator, width: int | None = None,
                        pad: int = -1) -> torch.Tensor:
    """Disjoint random block ids per sequence (consecutive slices of one permutation),
    right-padded with `pad` to `width` columns."""
    need = [math.ceil(c / block_size) for c in context_lens]
    width = width or max(max(need), 1)
    assert sum(need) <= num_blocks
    perm = torch.randperm(num_blocks, generator=g)
    bt = torch.full((len(context_lens), width), pad, dtype=torch.int32)
    pos = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[pos:pos + n].to(torch.int32)
        pos += n
    return bt


def bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bitwise equality of two bf16 tensors (NaN payloads included)."""
    return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


def relocate_pages(k_cache: torch.Tensor, v_cache: torch.Tensor, block_tables: torch.Tensor,
                   g: torch.Generator) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The same logical caches with every page moved to another physical block id: page p
    becomes page perm[p], and the table entries are renumbered to match (padding kept)."""
    nb = k_cache.shape[0]
    perm = torch.randperm(nb, generator=g)
    k2 = torch.empty_like(k_cache.contiguous())
    v2 = torch.empty_like(v_cache.contiguous())
    k2[perm] = k_cache
    v2[perm] = v_cache
    bt2 = block_tables.clone()
    valid = bt2 >= 0
    bt2[valid] = perm[bt2[valid].long()].to(torch.int32)
    return k2, v2, bt2
