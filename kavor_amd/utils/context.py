"""Per-step batch metadata shared by every attention layer.

Same contract as kavor/utils/context.py:5-32: the model runner publishes one Context
per forward pass with set_context(), attention layers read it with get_context(), and
models never receive it as an argument.  Device tensors are int32 except where noted;
max_seqlen_q/k are host ints (they size the prefill grid).  The three linear-attention
fields are kept so callers written against the reference construct it unchanged; the
paged KV path does not read them.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(slots=True)
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    linear_slot_ids: torch.Tensor | None = None
    linear_cache_slot_ids: torch.Tensor | None = None
    states_store_flags: torch.Tensor | None = None


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(is_prefill, cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=0, max_seqlen_k=0,
                slot_mapping=None, context_lens=None, block_tables=None, linear_slot_ids=None,
                linear_cache_slot_ids=None, states_store_flags=None) -> None:
    global _CONTEXT
    _CONTEXT = Context(is_prefill, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                       slot_mapping, context_lens, block_tables, linear_slot_ids,
                       linear_cache_slot_ids, states_store_flags)


def reset_context() -> None:
    global _CONTEXT
    _CONTEXT = Context()
