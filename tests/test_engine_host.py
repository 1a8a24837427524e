"""Host-side engine: Sequence, BlockManager and Scheduler (CPU only).

The scenarios and expected numbers restate the reference's own CPU tests for the
full-attention path: tests/test_sequence.py:9-27 and :81-87, tests/test_block_manager.py:25-173
and tests/test_scheduler.py:27-175.  Pages are 4 tokens so a few dozen tokens cover
multi-block cases.  The scheduler is driven without a model: every step "samples" a
fixed token 5 and eos is 0.
"""

from types import SimpleNamespace

import pytest

from kavor_amd.engine.block_manager import BlockManager
from kavor_amd.engine.scheduler import Scheduler
from kavor_amd.engine.sequence import Sequence, SequenceStatus
from kavor_amd.sampling_params import SamplingParams

BS = 4


@pytest.fixture(autouse=True)
def small_block_size(monkeypatch):
    monkeypatch.setattr(Sequence, "block_size", BS)


def make_seq(token_ids, *, temperature=1.0, max_tokens=64, ignore_eos=False):
    return Sequence(list(token_ids), SamplingParams(temperature=temperature, max_tokens=max_tokens,
                                                    ignore_eos=ignore_eos))


def make_config(**overrides):
    values = dict(max_num_seqs=8, max_num_batched_tokens=256, eos=0, kvcache_block_size=BS,
                  num_kvcache_blocks=64)
    values.update(overrides)
    return SimpleNamespace(**values)


def prefill_whole(bm, seq):
    """One single-chunk prefill: allocate, then key the full blocks (postprocess's first half)."""
    cached = bm.can_allocate_prefill(seq)
    assert cached != -1
    bm.allocate_prefill(seq, cached)
    seq.num_scheduled_tokens = seq.num_tokens - seq.num_cached_tokens
    bm.hash_blocks(seq)
    seq.num_cached_tokens += seq.num_scheduled_tokens
    seq.num_scheduled_tokens = 0


def drive(sched, token=5, max_steps=1000):
    steps = []
    while not sched.is_finished():
        batch, is_prefill = sched.schedule()
        assert batch
        sched.postprocess(batch, [token] * len(batch), is_prefill)
        steps.append(is_prefill)
        assert len(steps) < max_steps, "scheduler did not converge"
    return steps


# ------------------------------------------------------------------ sequence

def test_block_math():
    seq = make_seq(range(10))
    assert seq.num_blocks == 3
    assert seq.block(0) == [0, 1, 2, 3]
    assert seq.block(1) == [4, 5, 6, 7]
    assert seq.block(2) == [8, 9]
    assert seq.last_block_num_tokens == 2
    assert len(seq) == 10
    with pytest.raises(IndexError):
        seq.block(3)


def test_append_token_updates_state():
    seq = make_seq([1, 2, 3])
    seq.append_token(7)
    assert seq.num_tokens == 4 and seq.last_token == 7
    assert seq.num_completion_tokens == 1
    assert seq.prompt_token_ids == [1, 2, 3]
    assert seq.completion_token_ids == [7]


def test_status_lifecycle():
    seq = make_seq([1])
    assert seq.status == SequenceStatus.WAITING and not seq.is_finished
    seq.status = SequenceStatus.FINISHED
    assert seq.is_finished


def test_sampling_params_allow_greedy_and_reject_negative():
    assert SamplingParams(temperature=0.0).temperature == 0.0
    with pytest.raises(ValueError):
        SamplingParams(temperature=-0.1)
    with pytest.raises(ValueError):
        SamplingParams(max_tokens=0)


# ------------------------------------------------------------------ block manager

def test_allocate_and_deallocate_roundtrip():
    bm = BlockManager(num_blocks=8, block_size=BS)
    ids = [bm.allocate_block() for _ in range(8)]
    assert sorted(ids) == list(range(8)) and not bm.free_block_ids
    with pytest.raises(IndexError):
        bm.allocate_block()
    for block_id in ids:
        bm.blocks[block_id].ref_count = 0
        bm.deallocate_block(block_id)
    assert len(bm.free_block_ids) == 8


def test_hash_chains_parent_and_tokens():
    h1 = BlockManager.hash_block_tokens(None, [1, 2, 3, 4])
    assert h1 == BlockManager.hash_block_tokens(None, [1, 2, 3, 4])
    assert h1 != BlockManager.hash_block_tokens(None, [1, 2, 3, 5])
    assert h1 != BlockManager.hash_block_tokens(h1, [1, 2, 3, 4])
    # token ids are hashed as 64-bit values, so large ids do not collide with small ones
    assert (BlockManager.hash_block_tokens(None, [2**32 + 1])
            != BlockManager.hash_block_tokens(None, [1]))


def test_prefix_cache_reuses_finished_prefix():
    bm = BlockManager(num_blocks=16, block_size=BS)
    seq1 = make_seq(range(12))                  # 3 full blocks
    prefill_whole(bm, seq1)
    reused = seq1.block_table[:2]
    bm.deallocate(seq1)
    assert seq1.block_table == []

    seq2 = make_seq(range(12))                  # the last block is never taken from the cache
    cached = bm.can_allocate_prefill(seq2)
    assert cached == 2
    bm.allocate_prefill(seq2, cached)
    assert seq2.block_table[:2] == reused
    assert seq2.num_cached_tokens == 8
    assert all(bm.blocks[b].ref_count == 1 for b in reused)
    assert bm.prefix_cache_hit_tokens == 8
    assert bm.prefix_cache_prompt_tokens == 24


def test_prefix_cache_hits_only_up_to_divergence():
    bm = BlockManager(num_blocks=16, block_size=BS)
    seq1 = make_seq(range(12))
    prefill_whole(bm, seq1)
    bm.deallocate(seq1)
    seq2 = make_seq([0, 1, 2, 3, 40, 41, 42, 43, 8, 9, 10, 11])
    assert bm.can_allocate_prefill(seq2) == 1


def test_last_block_of_shorter_prompt_is_reusable():
    bm = BlockManager(num_blocks=16, block_size=BS)
    seq1 = make_seq(range(8))                   # 2 full blocks, both keyed
    prefill_whole(bm, seq1)
    bm.deallocate(seq1)
    assert bm.can_allocate_prefill(make_seq(range(12))) == 2


def test_hash_entry_with_mismatched_tokens_is_rejected():
    bm = BlockManager(num_blocks=16, block_size=BS)
    seq1 = make_seq(range(12))
    prefill_whole(bm, seq1)
    key1 = bm.blocks[seq1.block_table[1]].hash
    bm.hash_to_block_id[key1] = seq1.block_table[0]   # forged collision
    assert bm.can_allocate_prefill(make_seq(range(12))) == 1


def test_shared_prefix_with_running_seq_increases_refcount():
    bm = BlockManager(num_blocks=4, block_size=BS)
    seq1 = make_seq(range(12))
    prefill_whole(bm, seq1)                     # 3 pages used, 1 free
    seq2 = make_seq(range(12))
    cached = bm.can_allocate_prefill(seq2)
    assert cached == 2                          # needs only 1 new page
    bm.allocate_prefill(seq2, cached)
    assert not bm.free_block_ids
    shared = seq1.block_table[:2]
    assert all(bm.blocks[b].ref_count == 2 for b in shared)
    bm.deallocate(seq1)
    assert all(bm.blocks[b].ref_count == 1 and b in bm.used_block_ids for b in shared)
    bm.deallocate(seq2)
    assert len(bm.free_block_ids) == 4


def test_can_allocate_prefill_reports_shortage():
    bm = BlockManager(num_blocks=2, block_size=BS)
    assert bm.can_allocate_prefill(make_seq(range(12))) == -1


def test_allocate_block_evicts_stale_hash_entry():
    bm = BlockManager(num_blocks=16, block_size=BS)
    seq1 = make_seq(range(12))
    prefill_whole(bm, seq1)
    block_id = seq1.block_table[0]
    key = bm.blocks[block_id].hash
    bm.deallocate(seq1)
    assert bm.hash_to_block_id[key] == block_id      # free but still reusable
    bm.free_block_ids.remove(block_id)
    bm.free_block_ids.appendleft(block_id)
    assert bm.allocate_block() == block_id
    assert bm.blocks[block_id].hash is None
    assert key not in bm.hash_to_block_id


def test_may_append_block_grows_only_at_boundary():
    bm = BlockManager(num_blocks=8, block_size=BS)
    seq = make_seq(range(4))
    bm.allocate_prefill(seq, 0)
    seq.num_cached_tokens = 4
    seq.append_token(50)                        # token 5 starts block 2
    assert bm.can_append_block(seq)
    bm.may_append_block(seq)
    assert len(seq.block_table) == 2
    seq.append_token(51)
    bm.may_append_block(seq)
    assert len(seq.block_table) == 2


def test_partial_chunks_key_only_full_blocks():
    bm = BlockManager(num_blocks=8, block_size=BS)
    seq = make_seq(range(10))
    bm.allocate_prefill(seq, bm.can_allocate_prefill(seq))
    seq.num_scheduled_tokens = 3                # chunk ends inside block 0
    bm.hash_blocks(seq)
    assert all(bm.blocks[b].hash is None for b in seq.block_table)
    seq.num_cached_tokens, seq.num_scheduled_tokens = 3, 6   # ends inside block 2
    bm.hash_blocks(seq)
    assert [bm.blocks[b].hash is not None for b in seq.block_table] == [True, True, False]
    key0 = BlockManager.hash_block_tokens(None, [0, 1, 2, 3])
    assert bm.blocks[seq.block_table[1]].hash == BlockManager.hash_block_tokens(key0, [4, 5, 6, 7])


# ------------------------------------------------------------------ scheduler

def test_single_seq_prefill_then_decode():
    sched = Scheduler(make_config())
    seq = make_seq(range(6), max_tokens=3)
    sched.add(seq)
    batch, is_prefill = sched.schedule()
    assert is_prefill and batch == [seq]
    assert seq.num_scheduled_tokens == 6 and seq.status == SequenceStatus.RUNNING
    sched.postprocess(batch, [5], True)
    assert seq.num_tokens == 7 and seq.num_completion_tokens == 1
    batch, is_prefill = sched.schedule()
    assert not is_prefill and batch == [seq]
    assert seq.num_scheduled_tokens == 1 and not seq.is_prefill
    assert drive(sched) == [False, False]


def test_chunked_prefill_splits_by_token_budget():
    sched = Scheduler(make_config(max_num_batched_tokens=4))
    seq = make_seq(range(10), max_tokens=2)
    sched.add(seq)
    batch, is_prefill = sched.schedule()
    assert is_prefill and seq.num_scheduled_tokens == 4
    sched.postprocess(batch, [5], True)         # a pending chunk drops the sampled token
    assert seq.num_cached_tokens == 4 and seq.num_tokens == 10
    assert list(sched.waiting) == [seq]
    batch, _ = sched.schedule()
    assert seq.num_scheduled_tokens == 4
    sched.postprocess(batch, [5], True)
    assert seq.num_cached_tokens == 8
    batch, _ = sched.schedule()
    assert seq.num_scheduled_tokens == 2 and seq.status == SequenceStatus.RUNNING
    sched.postprocess(batch, [5], True)
    assert seq.num_completion_tokens == 1
    assert drive(sched) == [False]


def test_prefill_batches_multiple_seqs():
    sched = Scheduler(make_config(max_num_batched_tokens=32))
    seqs = [make_seq(range(i, i + 6), max_tokens=2) for i in range(3)]
    for s in seqs:
        sched.add(s)
    batch, is_prefill = sched.schedule()
    assert is_prefill and batch == seqs
    sched.postprocess(batch, [5] * 3, True)
    assert drive(sched) == [False]


def test_max_num_seqs_limits_batch():
    sched = Scheduler(make_config(max_num_seqs=1, max_num_batched_tokens=32))
    seq1, seq2 = make_seq([1, 2, 3, 4], max_tokens=2), make_seq([5, 6, 7, 8], max_tokens=2)
    sched.add(seq1)
    sched.add(seq2)
    _, is_prefill = sched.schedule()
    assert is_prefill
    sched.postprocess([seq1], [5], True)
    batch, is_prefill = sched.schedule()
    assert is_prefill and batch == [seq2]
    sched.postprocess(batch, [5], True)
    batch, is_prefill = sched.schedule()
    assert not is_prefill and batch == [seq1]
    sched.postprocess(batch, [5], False)
    assert drive(sched) == [False]


def test_head_of_line_blocking_on_budget():
    sched = Scheduler(make_config(max_num_batched_tokens=10))
    seq1, seq2 = make_seq(range(6), max_tokens=2), make_seq(range(10, 16), max_tokens=2)
    sched.add(seq1)
    sched.add(seq2)
    batch, is_prefill = sched.schedule()
    assert is_prefill and batch == [seq1]       # seq2 would need a chunk: it waits
    sched.postprocess(batch, [5], True)
    assert drive(sched)
    assert seq1.is_finished and seq2.is_finished


def test_preempt_on_block_exhaustion():
    sched = Scheduler(make_config(num_kvcache_blocks=4, max_num_batched_tokens=64))
    seq1, seq2 = make_seq([10], max_tokens=12), make_seq([20], max_tokens=12)
    sched.add(seq1)
    sched.add(seq2)
    preempted = []
    real = sched.preempt

    def spy(seq):
        preempted.append(seq)
        real(seq)

    sched.preempt = spy
    while not sched.is_finished():
        batch, is_prefill = sched.schedule()
        sched.postprocess(batch, [5] * len(batch), is_prefill)
        if preempted:
            break
    assert preempted == [seq2]                  # the newest running sequence is sacrificed
    assert seq2.status == SequenceStatus.WAITING and seq2.block_table == []
    assert seq2.num_cached_tokens == 0 and seq2.is_prefill
    assert list(sched.waiting)[0] is seq2
    drive(sched)
    assert seq1.is_finished and seq2.is_finished
    assert len(sched.block_manager.free_block_ids) == 4


def test_decode_finishes_on_eos_and_returns_pages():
    sched = Scheduler(make_config())
    seq = make_seq([1, 2, 3, 4], max_tokens=100)
    sched.add(seq)
    batch, _ = sched.schedule()
    sched.postprocess(batch, [5], True)
    batch, _ = sched.schedule()
    sched.postprocess(batch, [0], False)        # eos
    assert seq.is_finished and sched.is_finished()
    assert len(sched.block_manager.free_block_ids) == 64


def test_ignore_eos_runs_to_max_tokens():
    sched = Scheduler(make_config())
    seq = make_seq([1, 2, 3], max_tokens=4, ignore_eos=True)
    sched.add(seq)
    assert drive(sched, token=0) == [True, False, False, False]
    assert seq.completion_token_ids == [0, 0, 0, 0]


def test_finishes_on_max_tokens():
    sched = Scheduler(make_config())
    seq = make_seq(range(6), max_tokens=3)
    sched.add(seq)
    assert drive(sched) == [True, False, False]
    assert seq.num_completion_tokens == 3 and sched.is_finished()


def test_second_request_hits_prefix_through_scheduler():
    sched = Scheduler(make_config())
    seq1 = make_seq(range(13), max_tokens=1)
    sched.add(seq1)
    drive(sched)
    seq2 = make_seq(range(13), max_tokens=1)
    sched.add(seq2)
    batch, is_prefill = sched.schedule()
    assert is_prefill and seq2.num_cached_tokens == 12
    assert seq2.num_scheduled_tokens == 1
    assert seq2.stats.prefix_cache_hit_tokens == 12
    drive(sched)
    assert sched.block_manager.prefix_cache_hit_tokens == 12


@pytest.mark.parametrize("seed", range(12))
def test_random_workloads_keep_the_scheduler_invariants(seed):
    """Random prompts (some sharing prefixes), budgets, seat limits and small pools,
    driven to completion with ignore_eos.  Every step respects the token budget and the
    seats; a prefill step admits in queue order, and a partial chunk (of a prompt longer
    than the budget) is always the step's only sequence; a decode step schedules
    one token per sequence; every request ends with exactly max_tokens tokens, and all
    pages return to the free list."""
    import random

    rng = random.Random(seed)
    budget = rng.choice([8, 13, 32, 64])
    cfg = make_config(max_num_seqs=rng.choice([1, 2, 5, 8]), max_num_batched_tokens=budget,
                      num_kvcache_blocks=rng.choice([12, 24, 64]))
    sched = Scheduler(cfg)
    shared = [rng.randrange(1, 50) for _ in range(8)]
    seqs = []
    for _ in range(rng.randrange(1, 10)):
        n = rng.randrange(1, 30)
        toks = (shared[:rng.randrange(0, 9)] + [rng.randrange(1, 50) for _ in range(n)])[:29] or [7]
        seqs.append(make_seq(toks, max_tokens=rng.randrange(1, 12), ignore_eos=True))
    for s in seqs:
        sched.add(s)
    pool = cfg.num_kvcache_blocks
    steps = 0
    while not sched.is_finished():
        waiting_before = list(sched.waiting)
        batch, is_prefill = sched.schedule()
        assert batch and len(batch) <= cfg.max_num_seqs
        if is_prefill:
            assert sum(s.num_scheduled_tokens for s in batch) <= budget
            assert batch == waiting_before[:len(batch)]       # admitted in queue order
            partial = [s for s in batch if s.num_cached_tokens + s.num_scheduled_tokens < s.num_tokens]
            # only a step's sole sequence runs a partial chunk, and it fills the budget
            assert not partial or (batch == partial and batch[0].num_scheduled_tokens == budget)
        else:
            assert all(s.num_scheduled_tokens == 1 for s in batch)
            assert all(len(s.block_table) * BS >= s.num_tokens for s in batch)
        sched.postprocess(batch, [5] * len(batch), is_prefill)
        steps += 1
        assert steps < 5000
    assert all(s.is_finished and s.num_completion_tokens == s.max_tokens for s in seqs)
    assert len(sched.block_manager.free_block_ids) == pool
