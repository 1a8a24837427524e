"""The engine at the end-to-end workload's shape with a real decode batch: Qwen3-0.6B
(28 layers, hidden 1024, 16 q / 8 kv heads, head_dim 128, vocab 151936), random bf16
weights, 256-token pages and hipGraph decode over graphs of 1, 2, 4, 8, 16, 32, 48 and 64
rows (kavor/engine/model_runner.py:284-287).

44 requests with prompts of 100-1024 tokens drawn over the whole vocabulary (as the
benchmark workload draws them, kavor/benchs/bench.py:9-28) and output lengths spread
over 6-40 tokens run concurrently, so the decode batch shrinks from 44 to 1: it replays
the 48-row graph with 4 padding rows, then the 32-, 16- and 8-row graphs with padding,
down to a single row.  Every greedy token of every request is checked against a
full-sequence fp32-attention recomputation of the same weights
(tests/engine_reference.py), which uses no kernel of libkvpath.so.
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
NREQ = 44
TOL = 0.12  # as in test_engine_qwen3_shape.py: a wrong token sits about 2.5 below the maximum


def test_batch_of_44_through_padded_graphs_matches_reference(cuda_device):
    rng = np.random.default_rng(4444)
    vocab = SPEC.vocab_size
    lengths = rng.integers(100, 1025, NREQ).tolist()
    prompts = [rng.integers(0, vocab, n).tolist() for n in lengths]
    max_tokens = np.linspace(6, 40, NREQ).round().astype(int).tolist()
    rng.shuffle(max_tokens)
    llm = LLM(SPEC, kvcache_block_size=256, max_model_len=4096, max_num_seqs=64,
              max_num_batched_tokens=16384, gpu_memory_utilization=0.5, seed=0)
    try:
        assert sorted(llm.model_runner.graphs) == [1, 2, 4, 8, 16, 32, 48, 64]
        sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True) for m in max_tokens]
        outs = llm.generate(prompts, sps)
        assert [len(o["token_ids"]) for o in outs] == max_tokens
        decode_batches = {s["seqs"] for s in llm.step_stats if not s["prefill"]}
        # padded replays of the 48-, 32- and 16-row graphs, and the unpadded smallest ones
        assert max(decode_batches) == NREQ
        assert any(32 < b < 48 for b in decode_batches)
        assert any(16 < b < 32 for b in decode_batches)
        assert any(8 < b < 16 for b in decode_batches)
        assert 1 in decode_batches
        model = llm.model_runner.model
        worst = 0.0
        for p, o in zip(prompts, outs):
            worst = max(worst, check_greedy_tokens(model, p, o["token_ids"], TOL))
        print(f"{NREQ} requests, decode batches {sorted(decode_batches)}; largest shortfall below the "
              f"reference maximum: {worst:.4f} (tolerance {TOL})", flush=True)
    finally:
        llm.exit()
        torch.cuda.empty_cache()
