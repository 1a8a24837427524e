"""One request's token state, as the scheduler and the block manager see it.

Counterpart of kavor/engine/sequence.py (Sequence, SequenceStatus, SeqStats) restricted
to text-only full-attention models: the multimodal payload, the linear-attention state
blocks and the tensor-parallel pickling (sequence.py:143-160) are not part of the paged
KV path and are left out.

Block arithmetic follows sequence.py:115-120, 138-140: logical block i holds tokens
[i*block_size, (i+1)*block_size); block_table[i] is its physical page.  block_size is a
class attribute that the engine sets from its configuration before any Sequence is made.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum, auto
from itertools import count
from time import perf_counter
from typing import Sequence as _Seq

from kavor_amd.sampling_params import SamplingParams


class SequenceStatus(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


@dataclass
class SeqStats:
    """Engine-side timing of one request (sequence.py:18-56, text fields only)."""

    arrival_time: float = field(default_factory=perf_counter)
    prefill_start_time: float | None = None
    first_token_time: float | None = None
    finish_time: float | None = None
    prefix_cache_hit_tokens: int | None = None

    def mark_prefill_start(self) -> None:
        # a preempted sequence that is prefilled again keeps its first start time
        if self.prefill_start_time is None:
            self.prefill_start_time = perf_counter()

    def record_prefix_cache(self, hit_tokens: int) -> None:
        if self.prefix_cache_hit_tokens is None:
            self.prefix_cache_hit_tokens = hit_tokens


def _token_list(inputs) -> list[int]:
    """Accepts a list of token ids or any object with a `token_ids` attribute."""
    ids = getattr(inputs, "token_ids", inputs)
    return [int(t) for t in ids]


class Sequence:
    block_size = 256
    counter = count()

    def __init__(self, inputs: _Seq[int], sampling_params: SamplingParams | None = None):
        sp = sampling_params if sampling_params is not None else SamplingParams()
        token_ids = _token_list(inputs)
        if not token_ids:
            raise ValueError("a sequence needs at least one prompt token")
        self.seq_id = next(Sequence.counter)
        self.status = SequenceStatus.WAITING
        self.token_ids = token_ids
        self.last_token = token_ids[-1]
        self.num_tokens = len(token_ids)
        self.num_prompt_tokens = len(token_ids)
        # tokens whose K/V are already in the cache, and tokens in the current step
        self.num_cached_tokens = 0
        self.num_scheduled_tokens = 0
        self.is_prefill = True
        self.block_table: list[int] = []
        self.temperature = sp.temperature
        self.max_tokens = sp.max_tokens
        self.ignore_eos = sp.ignore_eos
        self.request_id: str | None = None
        self.stats = SeqStats()

    def __len__(self) -> int:
        return self.num_tokens

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def is_finished(self) -> bool:
        return self.status == SequenceStatus.FINISHED

    @property
    def num_completion_tokens(self) -> int:
        return self.num_tokens - self.num_prompt_tokens

    @property
    def prompt_token_ids(self) -> list[int]:
        return self.token_ids[:self.num_prompt_tokens]

    @property
    def completion_token_ids(self) -> list[int]:
        return self.token_ids[self.num_prompt_tokens:]

    @property
    def num_blocks(self) -> int:
        return -(-self.num_tokens // self.block_size)

    @property
    def last_block_num_tokens(self) -> int:
        return self.num_tokens - (self.num_blocks - 1) * self.block_size

    def block(self, i: int) -> list[int]:
        if not 0 <= i < self.num_blocks:
            raise IndexError(f"block {i} out of range [0, {self.num_blocks})")
        return self.token_ids[i * self.block_size:(i + 1) * self.block_size]

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1
