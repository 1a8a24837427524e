"""CPU oracle of Kavor's paged KV-cache path.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this
module, and only to compute expected answers (or as the timed CPU baseline): the product path is
kavor_amd/ over libkvpath.so and never calls into here.

Each function restates the reference algorithm it names (paths are relative to the
Kavor source tree):

  kv_append            store_kvcache_kernel / store_kvcache
                       kavor/layers/attention/flash_attention_kvcache.py:10-46
                       numpy over the raw bf16 bit patterns (a byte copy)
  paged_decode         flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
                       cache_seqlens, block_table, softmax_scale, causal=True)
                       flash_attention_kvcache.py:80-83 (flash-attn 2.8.3.post2,
                       setup.py:10): gather the first context_len tokens through the
                       block table, GQA head h -> kv head h // G, softmax(scale q k^T) v
                       in float32 (or float64) torch
  varlen_prefill       flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, ...,
                       causal=True, block_table) flash_attention_kvcache.py:73-79,
                       bottom-right causal mask (query i sees key j iff
                       j <= i + klen - qlen), rows with no visible key are zero
  prefill_metadata     ModelRunner.prepare_prefill slot / cu_seqlens construction,
                       kavor/engine/model_runner.py:385-446
  decode_metadata      ModelRunner.prepare_decode + prepare_block_tables,
                       model_runner.py:448-473
  page_views           CachePool._bind_attention_pages, kavor/engine/cache_pool.py:311-322
  sdpa_paged_decode /  the timed CPU baseline: the same gathers followed by
  sdpa_varlen_prefill  torch.nn.functional.scaled_dot_product_attention in the
                       reference's compute dtype (bf16), as a PyTorch-eager port of the
                       reference's CUDA path would run on host cores
  decode_bytes, append_bytes, prefill_flops, prefill_bytes
                       the algorithmic units of the measurements, counted by explicit
                       loops (token by token, pair by pair) for tests/test_bench_units.py,
                       which pins bench.py's closed forms against them

Pinning (tests/test_oracle.py): the reference ships no golden vectors for this path
(its tests cover other kernels), so every function is pinned by checks that a plausible
mistake fails: independent brute-force loops on tiny inputs, library routines
(torch SDPA with enable_gqa, is_causal for qlen == klen), closed forms (one-token
context returns V, zero query averages V, a dominant key selects its V row), invariants
(block renumbering, paged == dense on a packed copy) and raw-byte checks of the
interleaved page layout.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "bf16_bits", "kv_append", "paged_decode", "varlen_prefill", "prefill_metadata",
    "decode_metadata", "pad_block_tables", "page_views", "sdpa_paged_decode", "sdpa_varlen_prefill",
]


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    """numpy uint16 view (same memory, same strides) of a CPU bf16 tensor."""
    assert t.dtype == torch.bfloat16 and t.device.type == "cpu"
    return t.view(torch.int16).numpy().view(np.uint16)


# ---------------------------------------------------------------------------- append

def kv_append(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
              slot_mapping: np.ndarray) -> None:
    """store_kvcache_kernel (flash_attention_kvcache.py:10-34) on bf16 bit patterns.

    key / value: uint16 [N, Hkv, D]; k_cache / v_cache: uint16 [num_blocks, block_size,
    Hkv, D] views (any strides, written in place); slot_mapping: int [N].  Token i with
    slot s != -1 is copied to block s // block_size, offset s % block_size (the kernel's
    `block * BLOCK_STRIDE + offset_in_block * D` addressing, :30-32).  Rows are written
    in token order, so for duplicate slots the last token wins (the reference leaves the
    winner unspecified; tests never depend on it).
    """
    slots = np.asarray(slot_mapping).astype(np.int64)
    block_size = k_cache.shape[1]
    for i in np.flatnonzero(slots != -1):
        s = int(slots[i])
        blk, off = divmod(s, block_size)
        k_cache[blk, off] = key[i]
        v_cache[blk, off] = value[i]


# ---------------------------------------------------------------------------- attention

def _gather_tokens(cache: torch.Tensor, block_ids: torch.Tensor, ntok: int) -> torch.Tensor:
    """Logical tokens 0..ntok-1 of one sequence: token t = cache[block_ids[t // bs], t % bs]."""
    bs = cache.shape[1]
    nblk = (ntok + bs - 1) // bs
    ids = block_ids[:nblk].long()
    return cache[ids].reshape(nblk * bs, *cache.shape[2:])[:ntok]


def _attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
            mask: torch.Tensor | None) -> torch.Tensor:
    """q [Hq, Lq, D], k / v [Hkv, Lk, D] (Hq = G*Hkv) -> [Hq, Lq, D]; explicit softmax."""
    G = q.shape[0] // k.shape[0]
    k = k.repeat_interleave(G, dim=0)
    v = v.repeat_interleave(G, dim=0)
    s = torch.matmul(q, k.transpose(1, 2).contiguous()) * scale
    if mask is not None:
        s = s.masked_fill(~mask, float("-inf"))
    any_visible = torch.isfinite(s).any(dim=-1, keepdim=True)
    p = torch.softmax(s, dim=-1)
    p = torch.where(any_visible, p, torch.zeros_like(p))
    return torch.matmul(p, v)


def paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float,
                 dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """flash_attn_with_kvcache with one query token (flash_attention_kvcache.py:81-83).

    q [B, Hq, D]; caches [num_blocks, block_size, Hkv, D]; block_tables int [B, W];
    context_lens int [B] (tokens including the one just appended).  Returns [B, Hq, D]
    in `dtype`; a zero-length context returns zeros.  Block-table entries past
    ceil(ctx / block_size) are never read.  Runs on the device of its inputs (all on one
    device), so full-size checks can evaluate it in float32 on the GPU.
    """
    B, Hq, D = q.shape
    out = torch.zeros(B, Hq, D, dtype=dtype, device=q.device)
    for b in range(B):
        ctx = int(context_lens[b])
        if ctx <= 0:
            continue
        k = _gather_tokens(k_cache, block_tables[b], ctx).to(dtype).transpose(0, 1)
        v = _gather_tokens(v_cache, block_tables[b], ctx).to(dtype).transpose(0, 1)
        out[b] = _attend(q[b].to(dtype).unsqueeze(1), k, v, scale, None)[:, 0]
    return out


def varlen_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, scale: float,
                   causal: bool = True, block_tables: torch.Tensor | None = None,
                   dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """flash_attn_varlen_func (flash_attention_kvcache.py:76-79), bottom-right causal.

    q [Tq, Hq, D].  Dense mode (block_tables None): k / v [Tk, Hkv, D], sequence s owns
    rows cu_seqlens_k[s]:cu_seqlens_k[s+1].  Paged mode: k / v are caches and sequence s
    reads its klen_s logical tokens through block_tables[s].  Returns [Tq, Hq, D] on the
    device of q (inputs on one device; the cu_seqlens may be on the host or the device).
    """
    Tq, Hq, D = q.shape
    out = torch.zeros(Tq, Hq, D, dtype=dtype, device=q.device)
    cq = [int(x) for x in cu_seqlens_q]
    ck = [int(x) for x in cu_seqlens_k]
    for s in range(len(cq) - 1):
        qlen, klen = cq[s + 1] - cq[s], ck[s + 1] - ck[s]
        if qlen <= 0:
            continue
        if block_tables is None:
            ks, vs = k[ck[s]:ck[s + 1]], v[ck[s]:ck[s + 1]]
        else:
            ks = _gather_tokens(k, block_tables[s], klen)
            vs = _gather_tokens(v, block_tables[s], klen)
        qs = q[cq[s]:cq[s + 1]].to(dtype).transpose(0, 1)
        ks = ks.to(dtype).transpose(0, 1)
        vs = vs.to(dtype).transpose(0, 1)
        mask = None
        if causal:
            i = torch.arange(qlen, device=q.device).unsqueeze(1)
            j = torch.arange(klen, device=q.device).unsqueeze(0)
            mask = j <= i + (klen - qlen)
        out[cq[s]:cq[s + 1]] = _attend(qs, ks, vs, scale, mask).transpose(0, 1)
    return out


# ---------------------------------------------------------------------------- metadata

def prefill_metadata(block_tables: list[list[int]], num_cached: list[int],
                     num_scheduled: list[int], block_size: int) -> dict:
    """ModelRunner.prepare_prefill (model_runner.py:385-446), host lists only.

    For sequence s the new tokens are positions [num_cached, num_cached + num_scheduled);
    position p lands in slot block_table[p // bs] * bs + p % bs.  Block tables are
    produced (padded with -1) only when some sequence has cached tokens (:432-433).
    """
    slot_mapping, positions = [], []
    cu_q, cu_k = [0], [0]
    for bt, start, n in zip(block_tables, num_cached, num_scheduled):
        end = start + n
        positions.extend(range(start, end))
        cu_q.append(cu_q[-1] + n)
        cu_k.append(cu_k[-1] + end)
        for pos in range(start, end):
            slot_mapping.append(bt[pos // block_size] * block_size + pos % block_size)
    tables = pad_block_tables(block_tables) if cu_k[-1] > cu_q[-1] else None
    return dict(slot_mapping=slot_mapping, positions=positions, cu_seqlens_q=cu_q,
                cu_seqlens_k=cu_k, max_seqlen_q=max(np.diff(cu_q), default=0),
                max_seqlen_k=max(np.diff(cu_k), default=0), block_tables=tables)


def decode_metadata(block_tables: list[list[int]], seq_lens: list[int], block_size: int) -> dict:
    """ModelRunner.prepare_decode + prepare_block_tables (model_runner.py:448-473).

    The decoded token is the last one of the sequence: position len-1, slot
    block_table[-1] * bs + (tokens in the last block) - 1, context length len.
    Block tables are right-padded with -1 to the longest row.
    """
    slots, ctx, pos = [], [], []
    for bt, n in zip(block_tables, seq_lens):
        last_block_tokens = n - (len(bt) - 1) * block_size
        slots.append(bt[-1] * block_size + last_block_tokens - 1)
        ctx.append(n)
        pos.append(n - 1)
    return dict(slot_mapping=slots, context_lens=ctx, positions=pos,
                block_tables=pad_block_tables(block_tables))


def pad_block_tables(block_tables: list[list[int]]) -> list[list[int]]:
    """prepare_block_tables (model_runner.py:469-473): right-pad rows with -1."""
    width = max((len(bt) for bt in block_tables), default=0)
    return [list(bt) + [-1] * (width - len(bt)) for bt in block_tables]


def page_views(pool_page: torch.Tensor, block_size: int, num_kv_heads: int, head_dim: int,
               dtype: torch.dtype = torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor]:
    """CachePool._bind_attention_pages (cache_pool.py:311-322) for one layer's pool.

    pool_page is uint8 [num_blocks, page_bytes] with page_bytes = 2 * block_size *
    num_kv_heads * head_dim * itemsize; K occupies the first half of each page and V the
    second, so both views have block stride page_bytes / itemsize.
    """
    num_blocks, page_bytes = pool_page.shape
    flat = pool_page.view(dtype)
    block_elems = block_size * num_kv_heads * head_dim
    block_stride = page_bytes // flat.element_size()
    shape = (num_blocks, block_size, num_kv_heads, head_dim)
    strides = (block_stride, num_kv_heads * head_dim, head_dim, 1)
    base = flat.storage_offset()
    return flat.as_strided(shape, strides, base), flat.as_strided(shape, strides, base + block_elems)


# ---------------------------------------------------------------------------- CPU baseline

def sdpa_paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float) -> torch.Tensor:
    """Timed CPU baseline of paged decode: per-sequence gather + SDPA in q's dtype."""
    B, Hq, D = q.shape
    out = torch.zeros_like(q)
    for b in range(B):
        ctx = int(context_lens[b])
        if ctx <= 0:
            continue
        k = _gather_tokens(k_cache, block_tables[b], ctx).transpose(0, 1).unsqueeze(0)
        v = _gather_tokens(v_cache, block_tables[b], ctx).transpose(0, 1).unsqueeze(0)
        G = Hq // k.shape[1]
        k = k.repeat_interleave(G, dim=1)
        v = v.repeat_interleave(G, dim=1)
        out[b] = F.scaled_dot_product_attention(q[b].view(1, Hq, 1, D), k, v, scale=scale)[0, :, 0]
    return out


def torch_append(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 slot_mapping: torch.Tensor) -> None:
    """Timed CPU baseline of the append: PyTorch-eager index-put of the valid rows into
    the caches viewed as [num_blocks * block_size, Hkv * D] rows (block-stride aware)."""
    valid = slot_mapping >= 0
    slots = slot_mapping[valid].long()
    bs = k_cache.shape[1]
    for cache, src in ((k_cache, key), (v_cache, value)):
        rows = cache.reshape(cache.shape[0], bs, -1)
        rows[slots // bs, slots % bs] = src[valid].reshape(int(valid.sum()), -1)


def sdpa_varlen_prefill(q, k, v, cu_seqlens_q, cu_seqlens_k, scale, block_tables=None) -> torch.Tensor:
    """Timed CPU baseline of varlen prefill: per-sequence gather + masked SDPA."""
    out = torch.zeros_like(q)
    Hq = q.shape[1]
    cq = [int(x) for x in cu_seqlens_q]
    ck = [int(x) for x in cu_seqlens_k]
    for s in range(len(cq) - 1):
        qlen, klen = cq[s + 1] - cq[s], ck[s + 1] - ck[s]
        if block_tables is None:
            ks, vs = k[ck[s]:ck[s + 1]], v[ck[s]:ck[s + 1]]
        else:
            ks, vs = _gather_tokens(k, block_tables[s], klen), _gather_tokens(v, block_tables[s], klen)
        G = Hq // ks.shape[1]
        ks = ks.transpose(0, 1).repeat_interleave(G, dim=0).unsqueeze(0)
        vs = vs.transpose(0, 1).repeat_interleave(G, dim=0).unsqueeze(0)
        i = torch.arange(qlen).unsqueeze(1)
        j = torch.arange(klen).unsqueeze(0)
        mask = j <= i + (klen - qlen)
        qs = q[cq[s]:cq[s + 1]].transpose(0, 1).unsqueeze(0)
        out[cq[s]:cq[s + 1]] = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=mask, scale=scale)[0].transpose(0, 1)
    return out


def decode_bytes(context_lens, num_q_heads: int, num_kv_heads: int, head_dim: int,
                 block_size: int, elem: int = 2) -> int:
    """Algorithmic HBM bytes of one paged-decode launch: every valid K and V element of
    every sequence once, q and o once, plus context_lens and the block-table entries read."""
    ctx = [int(c) for c in context_lens]
    kv = sum(ctx) * num_kv_heads * head_dim * elem * 2
    qo = len(ctx) * num_q_heads * head_dim * elem * 2
    meta = len(ctx) * 4 + sum(math.ceil(c / block_size) for c in ctx) * 4
    return kv + qo + meta


def fused_decode_bytes(context_lens, num_q_heads: int, num_kv_heads: int, head_dim: int,
                       block_size: int, elem: int = 2) -> int:
    """Algorithmic HBM bytes of one one-launch decode step (q/k norm + RoPE + append +
    paged decode), counted sequence by sequence (contexts of at least one token): its qkv
    row, fp32 cos/sin row, slot and context length read; its block-table entries read; the
    K and V of its cached tokens (all but the new one) read; the new token's K and V and
    its output written."""
    total = 0
    for c in (int(x) for x in context_lens):
        total += (num_q_heads + 2 * num_kv_heads) * head_dim * elem + head_dim * 4 + 4 + 4
        total += math.ceil(c / block_size) * 4
        total += (c - 1) * num_kv_heads * head_dim * elem * 2
        total += num_kv_heads * head_dim * elem * 2 + num_q_heads * head_dim * elem
    return total


def append_bytes(slot_mapping, num_kv_heads: int, head_dim: int, elem: int = 2) -> int:
    """Algorithmic HBM bytes of one KV append: read + write of K and V for each valid
    token, plus the slot_mapping read."""
    slots = np.asarray(slot_mapping)
    n_valid = int((slots != -1).sum())
    return n_valid * num_kv_heads * head_dim * elem * 4 + slots.size * 4


def prefill_flops(cu_seqlens_q, cu_seqlens_k, num_q_heads: int, head_dim: int, causal: bool = True) -> int:
    """Algorithmic flops of varlen prefill over the unmasked (query, key) pairs:
    4 * Hq * D per pair (QK^T and PV multiply-adds)."""
    cq = [int(x) for x in cu_seqlens_q]
    ck = [int(x) for x in cu_seqlens_k]
    pairs = 0
    for s in range(len(cq) - 1):
        qlen, klen = cq[s + 1] - cq[s], ck[s + 1] - ck[s]
        if not causal:
            pairs += qlen * klen
            continue
        for i in range(qlen):
            pairs += max(0, min(klen, i + klen - qlen + 1))
    return 4 * num_q_heads * head_dim * pairs


def prefill_bytes(cu_seqlens_q, cu_seqlens_k, num_q_heads: int, num_kv_heads: int, head_dim: int,
                  block_tables=None, block_size: int = 0) -> int:
    """Algorithmic HBM bytes of a varlen prefill call, counted token by token: q and o
    rows (read and written once), each distinct key read once as a K and a V row (with
    block tables, logical token t of sequence s is the physical (block_tables[s][t // bs],
    t % bs), so tokens of shared prefix pages count once), and 4 bytes per cu_seqlens
    entry and per block-table entry the sequences need."""
    cq = [int(x) for x in cu_seqlens_q]
    ck = [int(x) for x in cu_seqlens_k]
    q_rows = sum(cq[s + 1] - cq[s] for s in range(len(cq) - 1))
    keys = set()
    entries = 0
    for s in range(len(ck) - 1):
        klen = ck[s + 1] - ck[s]
        for t in range(klen):
            keys.add((s, t) if block_tables is None else (int(block_tables[s][t // block_size]), t % block_size))
        if block_tables is not None:
            entries += (klen + block_size - 1) // block_size
    row = head_dim * 2
    return (q_rows * num_q_heads * row * 2 + len(keys) * num_kv_heads * row * 2
            + 4 * (len(cq) + len(ck)) + 4 * entries)
