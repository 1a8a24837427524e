"""Continuous-batching scheduler for the paged KV path.

Observable behaviour of Scheduler.schedule_full_attention / preempt / postprocess in
kavor/engine/scheduler.py:113-178 (the linear-attention variant, :34-111, and its
snapshot clamp, :181-195, are not part of the paged KV path), which the restated
reference tests pin (tests/test_engine_host.py):

- a step is either a prefill step or a decode step, and prefill has priority;
- prefill admission walks the waiting queue in arrival order under two limits, the
  step's token budget (max_num_batched_tokens) and its sequence seats (max_num_seqs).
  Admission stops at the first sequence whose pages cannot be allocated, and at the
  first one whose remaining prompt exceeds the budget left, unless it would be the
  step's only sequence, in which case it runs a budget-sized chunk (head-of-line
  blocking, :131-132);
- a sequence moves from waiting to running when its last prompt chunk is scheduled;
- a decode step takes running sequences in order, one token each; one that needs a
  fresh page when none is free reclaims pages by preempting the newest running
  sequence, or itself when no other is left (:155-167).  A preempted sequence drops its
  pages and goes back to the head of the waiting queue to be recomputed;
- after a step, the blocks it filled are keyed for the prefix cache, num_cached_tokens
  advances, and the sampled token is appended unless a prompt chunk is still pending; a
  sequence finishes on EOS (unless ignore_eos) or after max_tokens completion tokens.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass

from kavor_amd.engine.block_manager import BlockManager
from kavor_amd.engine.sequence import Sequence, SequenceStatus


@dataclass
class StepBudget:
    """What is left of one step's limits while sequences are admitted."""

    tokens: int
    seats: int

    def take(self, num_tokens: int) -> None:
        self.tokens -= num_tokens
        self.seats -= 1


class Scheduler:

    def __init__(self, config):
        self.max_num_seqs = config.max_num_seqs
        self.max_num_batched_tokens = config.max_num_batched_tokens
        self.eos = config.eos
        self.block_size = config.kvcache_block_size
        self.block_manager = BlockManager(config.num_kvcache_blocks, config.kvcache_block_size)
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()

    def is_finished(self) -> bool:
        return not self.waiting and not self.running

    def add(self, seq: Sequence) -> None:
        self.waiting.append(seq)

    # ------------------------------------------------------------------ a step

    def schedule(self) -> tuple[list[Sequence], bool]:
        """The next step's sequences and whether it is a prefill step."""
        prefill = self._admit_prefill()
        if prefill:
            return prefill, True
        decode = self._admit_decode()
        assert decode, "nothing to schedule: the page pool cannot hold a single sequence"
        return decode, False

    # ------------------------------------------------------------------ prefill

    def _prompt_tokens_left(self, seq: Sequence) -> tuple[int, int] | None:
        """(prompt tokens `seq` still has to compute if admitted now, prefix blocks it
        can take from the cache): after its cached prefix for a sequence without pages,
        else after its earlier chunks (no blocks to take).  None when the pool cannot
        supply its pages."""
        if seq.block_table:
            return seq.num_tokens - seq.num_cached_tokens, 0
        cached_blocks = self.block_manager.can_allocate_prefill(seq)
        if cached_blocks < 0:
            return None
        return seq.num_tokens - cached_blocks * self.block_size, cached_blocks

    def _take_pages(self, seq: Sequence, cached_blocks: int) -> None:
        """Allocates a fresh sequence's pages, taking its cached prefix blocks."""
        self.block_manager.allocate_prefill(seq, cached_blocks)
        seq.stats.mark_prefill_start()
        seq.stats.record_prefix_cache(seq.num_cached_tokens)

    def _admit_prefill(self) -> list[Sequence]:
        budget = StepBudget(self.max_num_batched_tokens, self.max_num_seqs)
        step: list[Sequence] = []
        for seq in list(self.waiting):
            if budget.seats == 0 or budget.tokens == 0:
                break
            plan = self._prompt_tokens_left(seq)
            if plan is None:
                break  # no pages for it; later arrivals wait behind it
            needed, cached_blocks = plan
            if needed > budget.tokens and step:
                break  # only a step's first sequence may run a partial chunk
            if not seq.block_table:
                self._take_pages(seq, cached_blocks)
            seq.num_scheduled_tokens = min(needed, budget.tokens)
            budget.take(seq.num_scheduled_tokens)
            step.append(seq)
            if seq.num_cached_tokens + seq.num_scheduled_tokens < seq.num_tokens:
                break  # a chunk: it stays at the head of the queue for the next step
            self.waiting.popleft()
            seq.status = SequenceStatus.RUNNING
            self.running.append(seq)
        return step

    # ------------------------------------------------------------------ decode

    def _reclaim_page_for(self, seq: Sequence) -> bool:
        """Frees pages, newest running sequence first, until `seq` can grow by one
        token.  Returns False when `seq` itself had to be preempted."""
        bm = self.block_manager
        while not bm.can_append_block(seq):
            victim = self.running.pop() if self.running else seq
            self.preempt(victim)
            if victim is seq:
                return False
        return True

    def _admit_decode(self) -> list[Sequence]:
        step: list[Sequence] = []
        while self.running and len(step) < self.max_num_seqs:
            seq = self.running.popleft()
            if not self._reclaim_page_for(seq):
                continue
            seq.num_scheduled_tokens = 1
            seq.is_prefill = False
            self.block_manager.may_append_block(seq)
            step.append(seq)
        # the step's sequences keep their places at the front of the running queue
        self.running.extendleft(reversed(step))
        return step

    def preempt(self, seq: Sequence) -> None:
        """Drops `seq`'s pages; it is recomputed from its tokens when admitted again."""
        seq.status = SequenceStatus.WAITING
        seq.is_prefill = True
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    # ------------------------------------------------------------------ after a step

    def _finished(self, seq: Sequence, token_id: int) -> bool:
        if seq.num_completion_tokens == seq.max_tokens:
            return True
        return not seq.ignore_eos and token_id == self.eos

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool) -> None:
        bm = self.block_manager
        for seq, token_id in zip(seqs, token_ids):
            bm.hash_blocks(seq)
            seq.num_cached_tokens += seq.num_scheduled_tokens
            seq.num_scheduled_tokens = 0
            chunk_pending = is_prefill and seq.num_cached_tokens < seq.num_tokens
            if chunk_pending:
                continue  # the token sampled after a partial prompt is discarded
            seq.append_token(token_id)
            if self._finished(seq, token_id):
                seq.status = SequenceStatus.FINISHED
                bm.deallocate(seq)
                self.running.remove(seq)
