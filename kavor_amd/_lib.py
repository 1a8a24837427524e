"""ctypes binding of libkvpath.so (declared in include/kvpath.h).

The library is the only compute path: if it is missing this module raises instead of
falling back to anything else.  Build it with ``python -m kavor_amd._build``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libkvpath.so")

KVP_OK = 0
KVP_EINVAL = -1
KVP_EUNSUPPORTED = -2
KVP_EWORKSPACE = -3

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_size_t = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/kvpath.h one to one.
SIGNATURES: dict[str, tuple] = {
    "kvp_last_error": (ctypes.c_char_p, []),
    "kvp_version": (ctypes.c_char_p, []),
    "kvp_append_bf16": (ctypes.c_int, [
        _c_void_p, _i64, _i64,            # key, key_tok_stride, key_head_stride
        _c_void_p, _i64, _i64,            # value, value_tok_stride, value_head_stride
        _c_void_p, _c_void_p,             # k_cache, v_cache
        _i64, _i64, _i64, _i64,           # cache block/slot/head strides, num_cache_slots
        _c_void_p, _i32,                  # slot_mapping, num_tokens
        _i32, _i32, _i32,                 # num_kv_heads, head_dim, block_size
        _c_void_p,                        # stream
    ]),
    "kvp_decode_workspace_bytes": (_size_t, [_i32, _i32, _i32, _i32, _i32]),
    "kvp_paged_decode_bf16": (ctypes.c_int, [
        _c_void_p, _i64, _i64,            # q, q_seq_stride, q_head_stride
        _c_void_p, _c_void_p,             # k_cache, v_cache
        _i64, _i64, _i64, _i32,           # cache block/slot/head strides, num_cache_blocks
        _c_void_p, _i64,                  # block_tables, block_table_stride
        _c_void_p, _i32,                  # context_lens, num_seqs
        _i32, _i32, _i32,                 # num_q_heads, num_kv_heads, head_dim
        _i32, _i32,                       # block_size, max_blocks_per_seq
        _f32,                             # softmax_scale
        _c_void_p, _i64, _i64,            # out, out_seq_stride, out_head_stride
        _c_void_p, _size_t, _c_void_p,    # workspace, workspace_bytes, stream
    ]),
    "kvp_paged_decode_fused_bf16": (ctypes.c_int, [
        _c_void_p, _i64,                  # qkv, qkv_tok_stride
        _c_void_p, _i32,                  # cos_sin, max_position
        _c_void_p, _c_void_p, _f32,       # q_norm_weight, k_norm_weight, eps
        _c_void_p, _c_void_p,             # k_cache, v_cache
        _i64, _i64, _i64, _i32,           # cache block/slot/head strides, num_cache_blocks
        _c_void_p,                        # slot_mapping
        _c_void_p, _i64,                  # block_tables, block_table_stride
        _c_void_p, _i32,                  # context_lens, num_seqs
        _i32, _i32, _i32,                 # num_q_heads, num_kv_heads, head_dim
        _i32, _i32, _f32,                 # block_size, max_blocks_per_seq, softmax_scale
        _c_void_p, _i64, _i64,            # out, out_seq_stride, out_head_stride
        _c_void_p, _size_t, _c_void_p,    # workspace, workspace_bytes, stream
    ]),
    "kvp_paged_decode_bf16_noalloc": (ctypes.c_int, [
        _c_void_p, _i64, _i64,            # q, q_seq_stride, q_head_stride
        _c_void_p, _c_void_p,             # k_cache, v_cache
        _i64, _i64, _i64, _i32,           # cache block/slot/head strides, num_cache_blocks
        _c_void_p, _i64,                  # block_tables, block_table_stride
        _c_void_p, _i32,                  # context_lens, num_seqs
        _i32, _i32, _i32,                 # num_q_heads, num_kv_heads, head_dim
        _i32, _i32,                       # block_size, max_blocks_per_seq
        _f32,                             # softmax_scale
        _c_void_p, _i64, _i64,            # out, out_seq_stride, out_head_stride
        _c_void_p,                        # stream
    ]),
    "kvp_varlen_prefill_bf16": (ctypes.c_int, [
        _c_void_p, _i64, _i64,            # q, q_tok_stride, q_head_stride
        _c_void_p, _i64, _i64, _i64,      # k, k_block_stride, k_tok_stride, k_head_stride
        _c_void_p, _i64, _i64, _i64,      # v, v_block_stride, v_tok_stride, v_head_stride
        _c_void_p, _i64,                  # block_tables, block_table_stride
        _i32, _i32, _i32,                 # num_cache_blocks, block_size, max_blocks_per_seq
        _c_void_p, _c_void_p,             # cu_seqlens_q, cu_seqlens_k
        _i32, _i32,                       # num_seqs, max_seqlen_q
        _i32, _i32, _i32,                 # num_q_heads, num_kv_heads, head_dim
        _f32, _i32,                       # softmax_scale, causal
        _c_void_p, _i64, _i64,            # out, out_tok_stride, out_head_stride
        _c_void_p, _size_t, _c_void_p,    # workspace, workspace_bytes, stream
    ]),
    "kvp_prefill_workspace_bytes": (_size_t, [_i32, _i32, _i32, _i32]),
    "kvp_rmsnorm_bf16": (ctypes.c_int, [
        _c_void_p, _i64, _i64,            # x, x_stride0, x_stride1
        _c_void_p, _i64, _i64,            # residual, residual_stride0, residual_stride1
        _c_void_p, _f32,                  # weight, eps
        _c_void_p, _i64, _i64,            # out, out_stride0, out_stride1
        _i32, _i32, _i32,                 # num_tokens, rows_per_token, cols
        _c_void_p,                        # stream
    ]),
    "kvp_qk_norm_rope_append_bf16": (ctypes.c_int, [
        _c_void_p, _i64,                  # qkv, qkv_tok_stride
        _c_void_p, _c_void_p, _i32,       # positions, cos_sin, max_position
        _c_void_p, _c_void_p, _f32,       # q_norm_weight, k_norm_weight, eps
        _c_void_p, _i64,                  # q_out, q_out_tok_stride
        _c_void_p, _c_void_p,             # k_cache, v_cache
        _i64, _i64, _i64, _i64,           # cache block/slot/head strides, num_cache_slots
        _c_void_p, _i32,                  # slot_mapping, num_tokens
        _i32, _i32, _i32, _i32,           # num_q_heads, num_kv_heads, head_dim, block_size
        _c_void_p,                        # stream
    ]),
    "kvp_qk_norm_rope_bf16": (ctypes.c_int, [
        _c_void_p, _i64,                  # qkv, qkv_tok_stride
        _c_void_p, _c_void_p, _i32,       # positions, cos_sin, max_position
        _c_void_p, _c_void_p, _f32,       # q_norm_weight, k_norm_weight, eps
        _c_void_p, _i64,                  # q_out, q_out_tok_stride
        _c_void_p, _i64,                  # k_out, k_out_tok_stride
        _i32, _i32, _i32, _i32,           # num_tokens, num_q_heads, num_kv_heads, head_dim
        _c_void_p,                        # stream
    ]),
    "kvp_silu_mul_bf16": (ctypes.c_int, [
        _c_void_p, _i64, _c_void_p, _i64,  # gate_up, gate_up_tok_stride, out, out_tok_stride
        _i32, _i32, _c_void_p,            # num_tokens, intermediate, stream
    ]),
    "kvp_argmax_workspace_bytes": (_size_t, [_i32]),
    "kvp_argmax_bf16": (ctypes.c_int, [
        _c_void_p, _i64, _i32, _i32,      # logits, row_stride, num_rows, vocab
        _c_void_p,                        # out (int64)
        _c_void_p, _size_t, _c_void_p,    # workspace, workspace_bytes, stream
    ]),
    "kvp_sample_bf16": (ctypes.c_int, [
        _c_void_p, _i64, _i32, _i32,      # logits, row_stride, num_rows, vocab
        _c_void_p, _c_void_p,             # temperatures (fp32), seed (int32, device)
        _c_void_p,                        # out (int64)
        _c_void_p, _size_t, _c_void_p,    # workspace, workspace_bytes, stream
    ]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Loads libkvpath.so once; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the HIP kernels with "
                    "`python -m kavor_amd._build` (there is no other compute path)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


class KVPathError(RuntimeError):
    """A libkvpath call rejected its arguments or failed to launch."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed ({code}): {message}")
        self.code = code


def check(fn: str, code: int) -> None:
    if code != KVP_OK:
        msg = lib().kvp_last_error().decode(errors="replace")
        raise KVPathError(fn, code, msg)


def version() -> str:
    return lib().kvp_version().decode()
