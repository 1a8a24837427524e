"""The engine at the end-to-end workload's shape: Qwen3-0.6B (28 layers, hidden 1024,
16 q / 8 kv heads, head_dim 128, vocab 151936) with random bf16 weights, 256-token
pages, hipGraph decode and a page pool sized from measured activation peaks
(num_kvcache_blocks = -1, kavor/engine/model_runner.py:329-383).

Every greedy token is checked against a full-sequence fp32-attention recomputation of
the same weights (tests/engine_reference.py), which uses no kernel of libkvpath.so.

The requests are laid out so that one run covers what the benchmark workload exercises
(kavor/benchs/bench.py:9-28 draws lengths 100-1024 over the vocabulary), with a token
budget of 2200 per step:
- request 0 (2600 tokens) is chunked at the budget, as the head of its step
  (kavor/engine/scheduler.py:128-139): a 2200-token prefill step (the q/k kernel's
  prefill-sized variant), then a chunk that starts at a cached length that is not a
  multiple of the page size;
- a second prefill step of more than 2048 tokens that mixes whole prompts;
- a prefix-cache hit inside one generate call: request 7 shares its first 512 tokens
  (two pages) with request 0 and is scheduled in the last prefill step, after request
  0's pages were keyed;
- a hit across generate calls on a repeated prompt, as in tests/test_e2e_gpu.py:54-70
  of the reference;
- decode batches of 8 shrinking to 1 as requests finish, replayed from the graphs of
  sizes 1, 2, 4 and 8 with padded rows.
"""

import numpy as np
import pytest
import torch

from kavor_amd.engine.llm_engine import LLM
from kavor_amd.engine.qwen3 import Qwen3Spec
from kavor_amd.sampling_params import SamplingParams
from tests.engine_reference import check_greedy_tokens

pytestmark = pytest.mark.gpu

SPEC = Qwen3Spec.qwen3_0_6b()
BLOCK = 256
PREFIX = 512
BUDGET = 2200
# Logits of these random weights have a standard deviation of about 0.6 and the top two
# of 151,936 are typically 0.1 apart; the bf16 kernels and the fp32 recomputation differ
# by a few 1e-2 after 28 layers.  A wrong token sits about 2.5 below the maximum.
TOL = 0.12


def _requests():
    rng = np.random.default_rng(2024)
    vocab = SPEC.vocab_size
    shared = rng.integers(0, vocab, PREFIX).tolist()
    lengths = [2600, 300, 1024, 900, 650, 100, 513, 812]
    prompts = []
    for i, n in enumerate(lengths):
        if i in (0, 7):
            prompts.append(shared + rng.integers(0, vocab, n - PREFIX).tolist())
        else:
            prompts.append(rng.integers(0, vocab, n).tolist())
    max_tokens = [24, 32, 28, 25, 30, 31, 26, 29]
    return prompts, max_tokens


@pytest.fixture(scope="module", params=["fused", "dropin"])
def llm(cuda_device, request):
    """Both caller orders: the fused q/k norm + RoPE + append kernel before attention over
    the pages, and the reference's order (Attention.forward appends, then dense or paged
    prefill)."""
    engine = LLM(SPEC, kvcache_block_size=BLOCK, max_model_len=4096, max_num_seqs=8,
                 max_num_batched_tokens=BUDGET, gpu_memory_utilization=0.5, seed=0,
                 attention_caller=request.param)
    yield engine
    engine.exit()
    torch.cuda.empty_cache()


def _check_all(llm, prompts, outs):
    model = llm.model_runner.model
    worst = 0.0
    for p, o in zip(prompts, outs):
        worst = max(worst, check_greedy_tokens(model, p, o["token_ids"], TOL))
    print(f"largest shortfall below the reference maximum: {worst:.4f} (tolerance {TOL})", flush=True)
    return worst


def test_pool_is_sized_from_measured_peaks(llm):
    runner = llm.model_runner
    assert llm.config.num_kvcache_blocks > 0
    layout = runner.pool.layout
    assert layout.num_blocks == llm.config.num_kvcache_blocks
    assert layout.num_pools == SPEC.num_hidden_layers and layout.page_bytes == 2 * BLOCK * 8 * 128 * 2
    free, total = torch.cuda.mem_get_info()
    # the pool plus everything else stays within the utilisation budget
    assert total - free <= 0.5 * total + 2**30
    assert sorted(runner.graphs) == [1, 2, 4, 8]


def test_full_shape_generation_matches_reference(llm):
    prompts, max_tokens = _requests()
    sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True) for m in max_tokens]
    hits_before = llm.scheduler.block_manager.prefix_cache_hit_tokens
    outs = llm.generate(prompts, sps)
    assert [len(o["token_ids"]) for o in outs] == max_tokens

    prefills = [s for s in llm.step_stats if s["prefill"]]
    decodes = [s for s in llm.step_stats if not s["prefill"]]
    # [r0 chunk] [r0 rest, r1, r2] [r3, r4, r5, r6] [r7 after its 512-token hit]
    assert [s["tokens"] for s in prefills] == [BUDGET, 400 + 300 + 1024, 900 + 650 + 100 + 513, 300]
    assert max(s["seqs"] for s in decodes) == 8 and min(s["seqs"] for s in decodes) == 1
    # request 7 found request 0's two shared pages in the last prefill step
    assert llm.scheduler.block_manager.prefix_cache_hit_tokens - hits_before == PREFIX
    hits = {r["seq_id"]: r["prefix_cache_hit_tokens"] for r in llm.request_stats}
    assert sorted(hits.values()).count(PREFIX) == 1

    _check_all(llm, prompts, outs)
    # greedy decoding of random weights settles into repetition loops, but the requests
    # do not collapse onto one token; and the checker rejects a wrong token
    tokens = [t for o in outs for t in o["token_ids"]]
    assert len(set(tokens)) >= 8
    bad = list(outs[1]["token_ids"])
    bad[5] = (bad[5] + 1) % SPEC.vocab_size
    with pytest.raises(AssertionError):
        check_greedy_tokens(llm.model_runner.model, prompts[1], bad, TOL)


def test_repeated_prompt_hits_the_prefix_cache(llm):
    prompts, _ = _requests()
    rng = np.random.default_rng(7)
    again = [prompts[2], rng.integers(0, SPEC.vocab_size, 333).tolist()]
    sp = SamplingParams(temperature=0.0, max_tokens=24, ignore_eos=True)
    hits_before = llm.scheduler.block_manager.prefix_cache_hit_tokens
    outs = llm.generate(again, sp)
    hits = llm.scheduler.block_manager.prefix_cache_hit_tokens - hits_before
    assert hits == 3 * BLOCK   # 1024 tokens: four pages, the last never taken from the cache
    _check_all(llm, again, outs)
