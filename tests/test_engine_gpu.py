"""End-to-end engine on the GPU with a small random Qwen3 (2 layers, 4/2 heads, D=128).

Greedy generations are checked token by token against a full-sequence fp32-attention
recomputation (tests/engine_reference.py): each generated token must be the reference
argmax up to a small logit tolerance.  The cases exercise what the paged path sees in
the engine: graph-replayed decode with padded batches, eager decode, prefix-cache hits
(paged prefill), chunked prefill and preemption with recomputation.
"""

import numpy as np
import pytest
import torch

from kavor_amd.engine.llm_engine import LLM
from kavor_amd.engine.qwen3 import Qwen3Spec
from kavor_amd.sampling_params import SamplingParams
from oracle import layers_oracle as lref
from tests.engine_reference import check_greedy_tokens

pytestmark = pytest.mark.gpu

TINY = Qwen3Spec(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                 num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                 max_position_embeddings=4096, eos_token_id=1)
TOL = 0.03   # logits have std ~0.3 with these weights; bf16 paths differ by ~1e-3


def _prompts(seed, lengths, vocab=TINY.vocab_size):
    rng = np.random.default_rng(seed)
    return [rng.integers(2, vocab, n).tolist() for n in lengths]


def _check(llm, prompts, outs):
    for p, o in zip(prompts, outs):
        check_greedy_tokens(llm.model_runner.model, p, o["token_ids"], TOL)


@pytest.fixture(scope="module")
def graph_llm(cuda_device):
    llm = LLM(TINY, kvcache_block_size=64, max_model_len=1024, num_kvcache_blocks=256,
              max_num_seqs=24, max_num_batched_tokens=1024, seed=0)
    yield llm
    llm.exit()


def test_graph_decode_matches_reference(graph_llm, monkeypatch):
    """Greedy decode steps take their tokens from the graph's LM head + argmax: the
    host-side sampler runs only for the prefill steps."""
    runner = graph_llm.model_runner
    calls = []
    sampler = runner.sampler
    monkeypatch.setattr(runner, "sampler", lambda *a: calls.append(1) or sampler(*a))
    prompts = _prompts(1, [1, 5, 63, 64, 65, 130, 300, 17, 200])
    sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True)
           for m in (12, 30, 7, 20, 64, 9, 25, 40, 3)]
    outs = graph_llm.generate(prompts, sps)
    assert len(calls) == sum(s["prefill"] for s in graph_llm.step_stats)
    assert [len(o["token_ids"]) for o in outs] == [sp.max_tokens for sp in sps]
    assert graph_llm.model_runner.graphs, "decode graphs were not captured"
    assert any(not s["prefill"] for s in graph_llm.step_stats)
    _check(graph_llm, prompts, outs)


def test_graph_decode_samples_at_temperature(graph_llm, monkeypatch):
    """A batch mixing greedy and T > 0 rows decodes through the graphs, whose sampler
    reads the rows' temperatures from the decode metadata and advances the device seed:
    each step's tokens equal the oracle's Gumbel-max draw over that step's logits with
    that seed (greedy rows: the argmax)."""
    runner = graph_llm.model_runner
    seen = []
    decode = runner._decode

    def spy(seqs):
        logits, sampled, temps = decode(seqs)
        if sampled is not None:
            torch.cuda.synchronize()
            seen.append((logits.cpu().clone(), sampled.cpu().clone(), temps.cpu().clone(),
                         int(runner.sampler.seed.item())))
        return logits, sampled, temps

    monkeypatch.setattr(runner, "_decode", spy)
    prompts = _prompts(7, [20, 33, 64, 5, 90])
    sps = [SamplingParams(temperature=t, max_tokens=8, ignore_eos=True) for t in (0.0, 0.8, 1.0, 1.5, 0.0)]
    outs = graph_llm.generate(prompts, sps)
    assert [len(o["token_ids"]) for o in outs] == [8] * 5
    assert len(seen) >= 5
    for logits, sampled, temps, seed in seen:
        t = temps.numpy()
        scores = lref.gumbel_scores(logits, t, seed)
        want = lref.first_argmax(scores)
        for r in range(len(want)):
            if sampled[r].item() != want[r]:
                a, b = scores[r, sampled[r].item()], scores[r, want[r]]
                assert abs(a - b) <= 4e-7 * max(1.0, abs(b)), (r, a, b)
    # the running order is the submission order
    assert np.allclose(seen[0][2].numpy(), [0.0, 0.8, 1.0, 1.5, 0.0])


def test_prefix_cache_hit_reuses_pages(graph_llm):
    base = _prompts(2, [200])[0]
    sp = SamplingParams(temperature=0.0, max_tokens=10, ignore_eos=True)
    first = graph_llm.generate([base], sp)
    hits_before = graph_llm.scheduler.block_manager.prefix_cache_hit_tokens
    prompts = [base + [5, 6, 7], base[:150]]
    outs = graph_llm.generate(prompts, sp)
    hits = graph_llm.scheduler.block_manager.prefix_cache_hit_tokens - hits_before
    assert hits == 192 + 128      # 3 and 2 full 64-token blocks
    _check(graph_llm, [base], first)
    _check(graph_llm, prompts, outs)


def test_chunked_prefill_and_eager_decode(cuda_device):
    llm = LLM(TINY, kvcache_block_size=64, max_model_len=1024, num_kvcache_blocks=64,
              max_num_seqs=4, max_num_batched_tokens=128, enforce_eager=True, seed=0)
    try:
        prompts = _prompts(3, [300, 90, 129])
        sps = SamplingParams(temperature=0.0, max_tokens=16, ignore_eos=True)
        outs = llm.generate(prompts, sps)
        chunks = [s for s in llm.step_stats if s["prefill"]]
        assert len(chunks) >= 5 and max(s["tokens"] for s in chunks) <= 128
        assert not llm.model_runner.graphs
        _check(llm, prompts, outs)
    finally:
        llm.exit()


def test_preemption_recomputes(cuda_device):
    # 6 pages of 64 tokens for three sequences that grow to 3 pages each
    llm = LLM(TINY, kvcache_block_size=64, max_model_len=512, num_kvcache_blocks=6,
              max_num_seqs=3, max_num_batched_tokens=512, seed=0)
    try:
        prompts = _prompts(4, [100, 110, 120])
        sps = SamplingParams(temperature=0.0, max_tokens=60, ignore_eos=True)
        outs = llm.generate(prompts, sps)
        prefills = sum(s["seqs"] for s in llm.step_stats if s["prefill"])
        assert prefills > 3, "expected at least one preempted sequence to be prefilled again"
        _check(llm, prompts, outs)
    finally:
        llm.exit()



def test_batches_beyond_the_largest_graph(cuda_device, monkeypatch):
    """With graphs captured only up to 4 sequences, a batch of 10 decodes eagerly and
    grows the decode workspace past what the graphs were captured with; as sequences
    finish the batch drops to 4 and below and the graphs replay on their own workspace.
    Every token of both phases must match the reference."""
    from kavor_amd.engine import model_runner
    from kavor_amd.layers import attention

    monkeypatch.setattr(model_runner, "MAX_GRAPH_BATCH", 4)
    ws = attention._workspaces.pop(cuda_device.index, None)
    if ws is not None:  # still used by graphs of other engines in this process
        attention._retired_workspaces.append(ws)
    llm = LLM(TINY, kvcache_block_size=64, max_model_len=1024, num_kvcache_blocks=128,
              max_num_seqs=16, max_num_batched_tokens=2048, seed=0)
    try:
        assert max(llm.model_runner.graphs) == 4
        captured = attention._workspaces[cuda_device.index].numel()
        prompts = _prompts(6, [70, 5, 130, 64, 200, 33, 90, 1, 150, 260])
        sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True)
               for m in (6, 9, 12, 15, 18, 21, 24, 30, 36, 40)]
        outs = llm.generate(prompts, sps)
        decode_sizes = [s["seqs"] for s in llm.step_stats if not s["prefill"]]
        assert max(decode_sizes) == 10 and min(decode_sizes) <= 4
        assert attention._workspaces[cuda_device.index].numel() > captured  # grown by eager steps
        _check(llm, prompts, outs)
    finally:
        llm.exit()

def test_sampling_with_temperature_runs_and_eos_stops(graph_llm):
    prompts = _prompts(5, [40, 80])
    outs = graph_llm.generate(prompts, [SamplingParams(temperature=0.8, max_tokens=32),
                                        SamplingParams(temperature=0.0, max_tokens=32)])
    for o in outs:
        toks = o["token_ids"]
        assert 1 <= len(toks) <= 32 and all(0 <= t < TINY.vocab_size for t in toks)
        if len(toks) < 32:
            assert toks[-1] == TINY.eos_token_id
    torch.cuda.synchronize()


def test_reference_design_comparator_is_correct(cuda_device, monkeypatch):
    """The benchmark's reference-design comparator (PyTorch-eager append and attention in
    place of the HIP path) generates reference-correct tokens too, with prefix-cache hits
    and chunked prefill in the mix, so the throughput comparison is between two correct
    engines."""
    import bench
    from kavor_amd.engine import qwen3

    monkeypatch.setattr(qwen3.Qwen3Attention, "forward", bench._eager_attention_forward)
    llm = LLM(TINY, kvcache_block_size=64, max_model_len=1024, num_kvcache_blocks=64,
              max_num_seqs=8, max_num_batched_tokens=256, enforce_eager=True, seed=0)
    try:
        base = _prompts(9, [150])[0]
        prompts = [base, base + [7, 8], _prompts(10, [300])[0], [3]]
        sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True) for m in (20, 9, 12, 30)]
        outs = llm.generate(prompts, sps)
        assert [len(o["token_ids"]) for o in outs] == [sp.max_tokens for sp in sps]
        _check(llm, prompts, outs)
    finally:
        llm.exit()


def test_dropin_caller_order_matches_reference(cuda_device, monkeypatch):
    """The reference's caller order (q/k norm + RoPE, then Attention.forward(q, k, v),
    which appends through store_kvcache): batches without a cached prefix run the dense
    varlen prefill over the fresh k / v, a batch with a prefix hit reads the pages, and
    decode replays graphs whose layers call the append kernel and the paged decode."""
    from kavor_amd.layers import attention

    modes, appends = [], []
    prefill, store = attention.varlen_prefill, attention.store_kvcache
    monkeypatch.setattr(attention, "varlen_prefill",
                        lambda *a, **kw: modes.append(kw.get("block_table") is not None) or prefill(*a, **kw))
    monkeypatch.setattr(attention, "store_kvcache", lambda *a: appends.append(a[0].shape[0]) or store(*a))
    llm = LLM(TINY, kvcache_block_size=64, max_model_len=1024, num_kvcache_blocks=128,
              max_num_seqs=8, max_num_batched_tokens=512, attention_caller="dropin", seed=0)
    try:
        assert llm.model_runner.graphs
        modes.clear()   # drop the warm-up and capture calls
        appends.clear()
        base = _prompts(11, [200])[0]
        first = [base, _prompts(12, [90])[0], _prompts(13, [600])[0]]   # 600 > budget: chunked
        sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True) for m in (20, 33, 9)]
        outs = llm.generate(first, sps)
        assert False in modes and True in modes  # dense first step, paged second chunk
        n_dense = modes.count(False)
        second = [base + [3, 4], _prompts(14, [70])[0]]   # mixed batch: one prefix hit
        outs2 = llm.generate(second, SamplingParams(temperature=0.0, max_tokens=12, ignore_eos=True))
        assert llm.scheduler.block_manager.prefix_cache_hit_tokens >= 192
        assert modes.count(False) == n_dense  # the mixed batch read the pages
        assert min(appends) >= 1
        _check(llm, first, outs)
        _check(llm, second, outs2)
    finally:
        llm.exit()


def test_separate_decode_launches_match_reference(cuda_device):
    """fused_decode off: the decode step runs the q/k norm + RoPE + append kernel and the
    paged decode as two launches (the layout of the previous engine); graphs, padding and
    prefix hits as in the default engine."""
    llm = LLM(TINY, kvcache_block_size=64, max_model_len=1024, num_kvcache_blocks=128,
              max_num_seqs=8, max_num_batched_tokens=1024, fused_decode=False, seed=0)
    try:
        assert not llm.model_runner.model.layers[0].self_attn.fused_decode
        prompts = _prompts(15, [3, 70, 129, 256, 40])
        sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True) for m in (20, 9, 33, 12, 5)]
        outs = llm.generate(prompts, sps)
        _check(llm, prompts, outs)
    finally:
        llm.exit()



@pytest.mark.parametrize("caller", ["fused", "dropin"])
def test_gqa_ratio_5_engine_matches_reference(cuda_device, caller):
    """Qwen3-14B's head ratio (40 query heads over 8 kv heads) at a small size, 10 over 2:
    prefill (tiles of 25 whole tokens), prefix hits, graph-replayed and eager decode
    through both callers, every token checked."""
    spec = Qwen3Spec(vocab_size=1024, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                     num_attention_heads=10, num_key_value_heads=2, head_dim=128,
                     max_position_embeddings=4096, eos_token_id=1)
    llm = LLM(spec, kvcache_block_size=64, max_model_len=1024, num_kvcache_blocks=128,
              max_num_seqs=8, max_num_batched_tokens=1024, attention_caller=caller, seed=0)
    try:
        assert llm.model_runner.graphs
        base = _prompts(21, [130], spec.vocab_size)[0]
        prompts = [base, _prompts(22, [1], spec.vocab_size)[0], _prompts(23, [77], spec.vocab_size)[0]]
        sps = [SamplingParams(temperature=0.0, max_tokens=m, ignore_eos=True) for m in (24, 10, 31)]
        outs = llm.generate(prompts, sps)
        again = [base + [5, 6, 7]]
        outs2 = llm.generate(again, SamplingParams(temperature=0.0, max_tokens=15, ignore_eos=True))
        assert llm.scheduler.block_manager.prefix_cache_hit_tokens >= 128
        for p, o in zip(prompts + again, outs + outs2):
            check_greedy_tokens(llm.model_runner.model, p, o["token_ids"], TOL)
    finally:
        llm.exit()


def test_copy_blocks_on_device_pages_feed_the_decode(cuda_device):
    """copy_blocks (cache_pool.py:142-149) on a device pool: the copied pages equal their
    sources byte for byte in every layer, the other pages keep their bytes, and paged
    decode over a block table that names the copies returns the same bits as over the
    originals."""
    from kavor_amd.engine.cache_pool import CachePool
    from kavor_amd.engine.qwen3 import Qwen3ForCausalLM
    from kavor_amd.layers.attention import paged_decode
    from oracle import kvpath_oracle as ref

    model = Qwen3ForCausalLM(TINY, cuda_device)
    hkv, D, bs = TINY.num_key_value_heads, TINY.head_dim, 64
    pool = CachePool(model, hkv, D, block_size=bs)
    pool.allocate(16, cuda_device)
    g = torch.Generator(device=cuda_device).manual_seed(3)
    pool.pools.view(torch.bfloat16).copy_(torch.randn(pool.pools.view(torch.bfloat16).shape, generator=g,
                                                      device=cuda_device, dtype=torch.bfloat16))
    before = pool.pools.clone()
    src, dst = [3, 7, 1], [10, 12, 14]
    pool.copy_blocks(src, dst)
    torch.cuda.synchronize()
    assert torch.equal(pool.pools[:, dst], before[:, src])
    others = [i for i in range(16) if i not in dst]
    assert torch.equal(pool.pools[:, others], before[:, others])
    kc, vc = ref.page_views(pool.pools[0], bs, hkv, D)
    q = torch.randn(2, TINY.num_attention_heads, D, generator=g, device=cuda_device, dtype=torch.bfloat16)
    ctx = torch.tensor([150, 100], dtype=torch.int32, device=cuda_device)
    bt_src = torch.tensor([[3, 7, 1], [1, 3, -1]], dtype=torch.int32, device=cuda_device)
    bt_dst = torch.tensor([[10, 12, 14], [14, 10, -1]], dtype=torch.int32, device=cuda_device)
    a = paged_decode(q, kc, vc, ctx, bt_src, D ** -0.5).clone()
    b = paged_decode(q, kc, vc, ctx, bt_dst, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.isfinite(a.float()).all()
