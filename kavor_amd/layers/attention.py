"""Drop-in attention boundary of the paged KV-cache path, backed by libkvpath.so.

Mirrors kavor/layers/attention/flash_attention_kvcache.py:
  store_kvcache(key, value, k_cache, v_cache, slot_mapping)      (:37-46)
  Attention(num_heads, head_dim, scale, num_kv_heads, num_kv_slots=1)
      .forward(q, k, v, slot=0)                                   (:49-84)
and replaces the two flash-attn calls it makes with
  paged_decode(...)    for flash_attn_with_kvcache(...)           (:80-83)
  varlen_prefill(...)  for flash_attn_varlen_func(...)            (:76-79)
which keep flash-attn's argument names and meaning.  Every function here only
validates layouts and forwards raw pointers and strides to the C ABI (include/kvpath.h)
on the current stream; nothing computes on the host and there is no fallback.
"""

from __future__ import annotations

import torch
from torch import nn

from kavor_amd._lib import check, lib
from kavor_amd.utils.context import get_context

__all__ = [
    "store_kvcache", "paged_decode", "paged_decode_fused", "varlen_prefill", "Attention",
    "reserve_decode_workspace", "decode_workspace_bytes",
    "reserve_prefill_workspace", "prefill_workspace_bytes",
    "flash_attn_with_kvcache", "flash_attn_varlen_func",
]


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_cuda_bf16(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA (HIP) tensor, got device {t.device}")
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {t.dtype}")


def _require_int32(name: str, t: torch.Tensor, device: torch.device) -> None:
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32, got {t.dtype}")
    if t.device != device:
        raise ValueError(f"{name} must live on {device}, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# ----------------------------------------------------------------------------- append

def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Writes key[i] / value[i] into slot slot_mapping[i] of k_cache / v_cache.

    Same contract and layout assertions as store_kvcache in
    kavor/layers/attention/flash_attention_kvcache.py:37-46: key/value are
    [N, num_kv_heads, head_dim] with contiguous heads (row strides may differ), the
    caches are [num_blocks, block_size, num_kv_heads, head_dim] views whose block
    stride may exceed block_size*num_kv_heads*head_dim (K/V interleaved pages), and
    slot -1 is skipped.  Bit-exact copy on the device.
    """
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    assert value.shape == key.shape
    assert k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride()
    assert k_cache.shape[2:] == (num_heads, head_dim)
    _require_cuda_bf16("key", key)
    _require_cuda_bf16("value", value)
    _require_cuda_bf16("k_cache", k_cache)
    _require_cuda_bf16("v_cache", v_cache)
    _require_int32("slot_mapping", slot_mapping, key.device)
    num_blocks, block_size = k_cache.shape[0], k_cache.shape[1]
    rc = lib().kvp_append_bf16(
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(),
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), num_blocks * block_size,
        slot_mapping.data_ptr(), N, num_heads, head_dim, block_size, _stream(key))
    check("kvp_append_bf16", rc)


# ----------------------------------------------------------------------------- decode

_workspaces: dict[int, torch.Tensor] = {}
# Outgrown workspaces are kept, never freed: a graph captured before the growth still
# launches the decode on the old buffer, and freed memory would be handed to new tensors.
_retired_workspaces: list[torch.Tensor] = []


def decode_workspace_bytes(max_num_seqs: int, num_q_heads: int, head_dim: int,
                           max_blocks_per_seq: int, block_size: int) -> int:
    return int(lib().kvp_decode_workspace_bytes(max_num_seqs, num_q_heads, head_dim,
                                                 max_blocks_per_seq, block_size))


def reserve_decode_workspace(max_num_seqs: int, num_q_heads: int, head_dim: int,
                             max_blocks_per_seq: int, block_size: int,
                             device: torch.device | str | int) -> torch.Tensor:
    """Allocates (or grows) the per-device decode workspace.  Call before graph capture
    with the largest batch a captured graph will use; an eager call that needs more grows
    the workspace without freeing the one the graphs hold."""
    nbytes = decode_workspace_bytes(max_num_seqs, num_q_heads, head_dim, max_blocks_per_seq, block_size)
    dev = torch.device(device) if not isinstance(device, int) else torch.device("cuda", device)
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    ws = _workspaces.get(dev.index)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                "the paged-decode workspace must be reserved before graph capture "
                f"({nbytes} bytes needed): call reserve_decode_workspace() first")
        if ws is not None:
            _retired_workspaces.append(ws)
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
        _workspaces[dev.index] = ws
    return ws


# ----------------------------------------------------------------------------- prefill workspace

_prefill_workspaces: dict[int, torch.Tensor] = {}


def prefill_workspace_bytes(num_seqs: int, max_seqlen_q: int, num_q_heads: int, num_kv_heads: int) -> int:
    return int(lib().kvp_prefill_workspace_bytes(num_seqs, max_seqlen_q, num_q_heads, num_kv_heads))


def reserve_prefill_workspace(num_seqs: int, max_seqlen_q: int, num_q_heads: int, num_kv_heads: int,
                              device: torch.device | str | int) -> torch.Tensor:
    """Allocates (or grows) the per-device prefill workspace: the work list of a launch
    (kvp_prefill_workspace_bytes).  A caller that captures prefill into a graph reserves
    the largest batch first; an eager call that needs more grows the workspace without
    freeing the one a graph holds."""
    nbytes = prefill_workspace_bytes(num_seqs, max_seqlen_q, num_q_heads, num_kv_heads)
    dev = torch.device(device) if not isinstance(device, int) else torch.device("cuda", device)
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    ws = _prefill_workspaces.get(dev.index)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                "the prefill workspace must be reserved before graph capture "
                f"({nbytes} bytes needed): call reserve_prefill_workspace() first")
        if ws is not None:
            _retired_workspaces.append(ws)
        ws = torch.empty(max(nbytes, 4096), dtype=torch.uint8, device=dev)
        _prefill_workspaces[dev.index] = ws
    return ws


def paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 cache_seqlens: torch.Tensor, block_table: torch.Tensor, softmax_scale: float,
                 causal: bool = True, out: torch.Tensor | None = None) -> torch.Tensor:
    """Paged decode attention, one query token per sequence.

    Argument meaning follows flash_attn_with_kvcache as called at
    kavor/layers/attention/flash_attention_kvcache.py:81-83: q is [B, 1, Hq, D] (or
    [B, Hq, D]), the caches are [num_blocks, block_size, Hkv, D], cache_seqlens int32 [B]
    counts the cached tokens including the one just appended, block_table int32
    [B, max_blocks] (entries past ceil(len/block_size) are never read).  Returns
    [B, 1, Hq, D] (or [B, Hq, D]) in bf16.  `causal` is accepted for signature
    compatibility; with one query token it changes nothing.
    """
    del causal
    if q.dim() == 4 and q.shape[1] == 1:
        q3, four_d = q[:, 0], True
    elif q.dim() == 3:
        q3, four_d = q, False
    else:
        raise ValueError(f"paged_decode takes one query token per sequence, got q of shape {tuple(q.shape)}")
    B, Hq, D = q3.shape
    _require_cuda_bf16("q", q3)
    _require_cuda_bf16("k_cache", k_cache)
    _require_cuda_bf16("v_cache", v_cache)
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share shape and strides")
    num_blocks, block_size, Hkv, Dk = k_cache.shape
    if Dk != D or k_cache.stride(3) != 1 or q3.stride(2) != 1:
        raise ValueError("head_dim mismatch or non-contiguous head_dim")
    _require_int32("cache_seqlens", cache_seqlens, q3.device)
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        raise ValueError("block_table must be an int32 [B, max_blocks] tensor with contiguous rows")
    if cache_seqlens.numel() < B or block_table.shape[0] < B:
        raise ValueError("cache_seqlens / block_table have fewer rows than q")
    if out is None:
        out3 = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=q3.device)
        out = out3.unsqueeze(1) if four_d else out3
    else:
        out3 = out[:, 0] if out.dim() == 4 else out
        if out3.shape != (B, Hq, D) or out3.dtype != torch.bfloat16 or out3.stride(2) != 1:
            raise ValueError("out must be bf16 [B, 1, Hq, D] or [B, Hq, D] with contiguous head_dim")
    max_blocks = block_table.shape[1]
    ws = reserve_decode_workspace(B, Hq, D, max_blocks, block_size, q3.device)
    rc = lib().kvp_paged_decode_bf16(
        q3.data_ptr(), q3.stride(0), q3.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(),
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), num_blocks,
        block_table.data_ptr(), block_table.stride(0),
        cache_seqlens.data_ptr(), B, Hq, Hkv, D, block_size, max_blocks,
        float(softmax_scale),
        out3.data_ptr(), out3.stride(0), out3.stride(1),
        ws.data_ptr(), ws.numel(), _stream(q3))
    check("kvp_paged_decode_bf16", rc)
    return out


def paged_decode_fused(qkv: torch.Tensor, cos_sin: torch.Tensor,
                       q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, eps: float,
                       num_q_heads: int, num_kv_heads: int, k_cache: torch.Tensor,
                       v_cache: torch.Tensor, slot_mapping: torch.Tensor, cache_seqlens: torch.Tensor,
                       block_table: torch.Tensor, softmax_scale: float,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """A Qwen3 decode step of one attention layer in one launch: q/k RMSNorm + RoPE of
    each sequence's new token from its qkv row, the append of its k / v at slot_mapping,
    and paged decode attention over cache_seqlens tokens (the last one being the new
    token).  Returns [B, Hq, 128] bf16.  The token's position is cache_seqlens - 1 and
    slot_mapping must hold the slot of that position, as the engine's decode metadata
    has them."""
    B = qkv.shape[0]
    D = k_cache.shape[-1]
    for name, t in (("qkv", qkv), ("k_cache", k_cache), ("v_cache", v_cache)):
        _require_cuda_bf16(name, t)
    if qkv.dim() != 2 or qkv.stride(1) != 1 or qkv.shape[1] != (num_q_heads + 2 * num_kv_heads) * D:
        raise ValueError("qkv must be [B, (Hq + 2 Hkv) * head_dim] with contiguous rows")
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share shape and strides")
    num_blocks, block_size, Hkv, _ = k_cache.shape
    if Hkv != num_kv_heads:
        raise ValueError("cache heads do not match num_kv_heads")
    for name, t in (("slot_mapping", slot_mapping), ("cache_seqlens", cache_seqlens)):
        _require_int32(name, t, qkv.device)
        if t.numel() < B:
            raise ValueError(f"{name} has fewer rows than qkv")
    if cos_sin.dtype != torch.float32 or not cos_sin.is_contiguous() or cos_sin.shape[1] != D:
        raise ValueError("cos_sin must be a contiguous fp32 [max_position, head_dim] table")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        raise ValueError("block_table must be an int32 [B, max_blocks] tensor with contiguous rows")
    if out is None:
        out = torch.empty(B, num_q_heads, D, dtype=torch.bfloat16, device=qkv.device)
    max_blocks = block_table.shape[1]
    ws = reserve_decode_workspace(B, num_q_heads, D, max_blocks, block_size, qkv.device)
    rc = lib().kvp_paged_decode_fused_bf16(
        qkv.data_ptr(), qkv.stride(0), cos_sin.data_ptr(), cos_sin.shape[0],
        q_norm_weight.data_ptr(), k_norm_weight.data_ptr(), float(eps),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        num_blocks, slot_mapping.data_ptr(), block_table.data_ptr(), block_table.stride(0),
        cache_seqlens.data_ptr(), B, num_q_heads, num_kv_heads, D, block_size, max_blocks,
        float(softmax_scale), out.data_ptr(), out.stride(0), out.stride(1),
        ws.data_ptr(), ws.numel(), _stream(qkv))
    check("kvp_paged_decode_fused_bf16", rc)
    return out


# ----------------------------------------------------------------------------- prefill

def varlen_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, max_seqlen_q: int,
                   cu_seqlens_q: torch.Tensor, max_seqlen_k: int, cu_seqlens_k: torch.Tensor,
                   softmax_scale: float, causal: bool = True,
                   block_table: torch.Tensor | None = None,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """Packed variable-length attention over dense or paged K/V (bf16 MFMA).

    Argument meaning follows flash_attn_varlen_func as called at
    kavor/layers/attention/flash_attention_kvcache.py:76-79: q is [Tq, Hq, D]; with
    block_table None, k / v are [Tk, Hkv, D] rows addressed through cu_seqlens_k; with
    a block_table they are the paged caches [num_blocks, block_size, Hkv, D].  The
    causal mask is bottom-right aligned.  Returns [Tq, Hq, D] bf16.  max_seqlen_k is
    accepted for signature compatibility (the kernel reads lengths on the device).
    """
    del max_seqlen_k
    Tq, Hq, D = q.shape
    _require_cuda_bf16("q", q)
    _require_cuda_bf16("k", k)
    _require_cuda_bf16("v", v)
    _require_int32("cu_seqlens_q", cu_seqlens_q, q.device)
    _require_int32("cu_seqlens_k", cu_seqlens_k, q.device)
    num_seqs = cu_seqlens_q.numel() - 1
    if cu_seqlens_k.numel() != num_seqs + 1:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must have the same length")
    if q.stride(2) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("head_dim must be contiguous in q, k and v")
    if out is None:
        out = torch.empty(Tq, Hq, D, dtype=torch.bfloat16, device=q.device)
    if block_table is None:
        if k.dim() != 3 or v.shape != k.shape:
            raise ValueError("dense k / v must be [Tk, Hkv, D] of equal shape")
        Hkv = k.shape[1]
        kstr = (0, k.stride(0), k.stride(1))
        vstr = (0, v.stride(0), v.stride(1))
        bt_ptr, bt_stride, num_blocks, block_size, max_blocks = 0, 0, 0, 0, 0
    else:
        if k.dim() != 4 or v.shape != k.shape:
            raise ValueError("paged k / v must be [num_blocks, block_size, Hkv, D] of equal shape")
        if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
            raise ValueError("block_table must be an int32 [B, max_blocks] tensor with contiguous rows")
        if block_table.shape[0] < num_seqs:
            raise ValueError("block_table has fewer rows than sequences")
        num_blocks, block_size, Hkv = k.shape[0], k.shape[1], k.shape[2]
        kstr = (k.stride(0), k.stride(1), k.stride(2))
        vstr = (v.stride(0), v.stride(1), v.stride(2))
        bt_ptr, bt_stride, max_blocks = block_table.data_ptr(), block_table.stride(0), block_table.shape[1]
    if k.shape[-1] != D:
        raise ValueError("head_dim mismatch between q and k")
    ws = reserve_prefill_workspace(num_seqs, int(max_seqlen_q), Hq, Hkv, q.device) if num_seqs else None
    rc = lib().kvp_varlen_prefill_bf16(
        q.data_ptr(), q.stride(0), q.stride(1),
        k.data_ptr(), *kstr,
        v.data_ptr(), *vstr,
        bt_ptr, bt_stride, num_blocks, block_size, max_blocks,
        cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), num_seqs, int(max_seqlen_q),
        Hq, Hkv, D, float(softmax_scale), 1 if causal else 0,
        out.data_ptr(), out.stride(0), out.stride(1),
        ws.data_ptr() if ws is not None else 0, ws.numel() if ws is not None else 0, _stream(q))
    check("kvp_varlen_prefill_bf16", rc)
    return out


# flash-attn spellings, so call sites written against flash_attn keep working.
flash_attn_with_kvcache = paged_decode
flash_attn_varlen_func = varlen_prefill


# ----------------------------------------------------------------------------- module

class Attention(nn.Module):
    """Paged-KV attention layer; same constructor, attributes and forward as
    kavor/layers/attention/flash_attention_kvcache.py:49-84.

    k_cache / v_cache are lists with one entry per KV slot (num_kv_slots); a page pool
    binds them by duck typing (kavor/engine/cache_pool.py:98-101, 311-322).  forward
    appends k / v when a cache is bound, then runs varlen prefill (paged when the
    context carries block tables) or paged decode, reading the global Context.
    """

    def __init__(self, num_heads, head_dim, scale, num_kv_heads, num_kv_slots: int = 1):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.num_kv_slots = num_kv_slots
        self.k_cache = [torch.tensor([]) for _ in range(num_kv_slots)]
        self.v_cache = [torch.tensor([]) for _ in range(num_kv_slots)]

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, slot: int = 0):
        context = get_context()
        k_cache, v_cache = self.k_cache[slot], self.v_cache[slot]
        if k_cache.numel() and v_cache.numel():
            store_kvcache(k, v, k_cache, v_cache, context.slot_mapping)
        if context.is_prefill:
            if context.block_tables is not None:  # prefix cache: attend over the pages
                k, v = k_cache, v_cache
            return self._prefill(q, k, v, context)
        return self._decode(q, k_cache, v_cache, context)

    def forward_cached(self, q: torch.Tensor, slot: int = 0):
        """Attention over the pages when the caller has already appended this step's k / v
        (the fused q/k-norm + RoPE + append kernel).  Prefill then always reads the pages,
        so the context must carry block tables."""
        context = get_context()
        k_cache, v_cache = self.k_cache[slot], self.v_cache[slot]
        if context.is_prefill:
            if context.block_tables is None:
                raise ValueError("forward_cached prefill reads the pages: the context needs block tables")
            return self._prefill(q, k_cache, v_cache, context)
        return self._decode(q, k_cache, v_cache, context)

    def _prefill(self, q, k, v, context):
        return varlen_prefill(q, k, v, max_seqlen_q=context.max_seqlen_q,
                              cu_seqlens_q=context.cu_seqlens_q,
                              max_seqlen_k=context.max_seqlen_k,
                              cu_seqlens_k=context.cu_seqlens_k,
                              softmax_scale=self.scale, causal=True,
                              block_table=context.block_tables)

    def _decode(self, q, k_cache, v_cache, context):
        return paged_decode(q.unsqueeze(1), k_cache, v_cache,
                            cache_seqlens=context.context_lens,
                            block_table=context.block_tables,
                            softmax_scale=self.scale, causal=True)
