"""Continuous-batching scheduler for the paged KV path.

Counterpart of Scheduler.schedule_full_attention / preempt / postprocess in
kavor/engine/scheduler.py:113-178 (the linear-attention variant, :34-111, and its
snapshot clamp, :181-195, are not part of the paged KV path):

- prefill first: waiting sequences are admitted in order while the step has token
  budget (max_num_batched_tokens) and sequence slots (max_num_seqs) left; a prompt
  longer than the remaining budget is chunked, but only when it is the first sequence
  of the step (head-of-line blocking, scheduler.py:131-132);
- a sequence leaves the waiting queue when its last prompt chunk is scheduled;
- otherwise a decode step takes up to max_num_seqs running sequences, one token each;
  a sequence that needs a new page when none is free preempts the newest running
  sequence (or itself), which returns to the head of the waiting queue to be
  recomputed (:155-167);
- postprocess keys the blocks the step completed, advances num_cached_tokens and
  appends the sampled token unless a prompt chunk is still pending; a sequence
  finishes on EOS (unless ignore_eos) or after max_tokens completion tokens.
"""

from __future__ import annotations

from collections import deque

from kavor_amd.engine.block_manager import BlockManager
from kavor_amd.engine.sequence import Sequence, SequenceStatus


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

    def schedule(self) -> tuple[list[Sequence], bool]:
        scheduled: list[Sequence] = []
        num_batched_tokens = 0
        bm = self.block_manager

        # prefill
        while self.waiting and len(scheduled) < self.max_num_seqs:
            seq = self.waiting[0]
            remaining = self.max_num_batched_tokens - num_batched_tokens
            if remaining == 0:
                break
            if not seq.block_table:
                num_cached_blocks = bm.can_allocate_prefill(seq)
                if num_cached_blocks == -1:
                    break
                num_tokens = seq.num_tokens - num_cached_blocks * self.block_size
            else:  # continuing a chunked prefill
                num_tokens = seq.num_tokens - seq.num_cached_tokens
            if remaining < num_tokens and scheduled:
                break
            if not seq.block_table:
                bm.allocate_prefill(seq, num_cached_blocks)
                seq.stats.mark_prefill_start()
                seq.stats.record_prefix_cache(seq.num_cached_tokens)
            seq.num_scheduled_tokens = min(num_tokens, remaining)
            num_batched_tokens += seq.num_scheduled_tokens
            if seq.num_cached_tokens + seq.num_scheduled_tokens == seq.num_tokens:
                seq.status = SequenceStatus.RUNNING
                self.waiting.popleft()
                self.running.append(seq)
            scheduled.append(seq)
        if scheduled:
            return scheduled, True

        # decode
        while self.running and len(scheduled) < self.max_num_seqs:
            seq = self.running.popleft()
            while not bm.can_append_block(seq):
                if self.running:
                    self.preempt(self.running.pop())
                else:
                    self.preempt(seq)
                    break
            else:
                seq.num_scheduled_tokens = 1
                seq.is_prefill = False
                bm.may_append_block(seq)
                scheduled.append(seq)
        assert scheduled, "nothing to schedule: the page pool cannot hold a single sequence"
        self.running.extendleft(reversed(scheduled))
        return scheduled, False

    def preempt(self, seq: Sequence) -> None:
        seq.status = SequenceStatus.WAITING
        seq.is_prefill = True
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool) -> None:
        bm = self.block_manager
        for seq, token_id in zip(seqs, token_ids):
            bm.hash_blocks(seq)
            seq.num_cached_tokens += seq.num_scheduled_tokens
            seq.num_scheduled_tokens = 0
            if is_prefill and seq.num_cached_tokens < seq.num_tokens:
                continue  # more prompt chunks to go; the sampled token is discarded
            seq.append_token(token_id)
            if ((not seq.ignore_eos and token_id == self.eos)
                    or seq.num_completion_tokens == seq.max_tokens):
                seq.status = SequenceStatus.FINISHED
                bm.deallocate(seq)
                self.running.remove(seq)
