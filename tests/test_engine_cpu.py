"""Engine pieces that run without a GPU: step metadata, page-pool layout, the Qwen3
layer arithmetic and the checkpoint round trip.

Step metadata is checked against the oracle's restatement of
ModelRunner.prepare_prefill / prepare_decode (kavor/engine/model_runner.py:385-473) on
sequences driven by the real scheduler; the pool views against the oracle's
CachePool binding (cache_pool.py:311-322).
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from kavor_amd.engine.cache_pool import CachePool
from kavor_amd.engine.metadata import decode_arrays, prefill_arrays
from kavor_amd.engine.qwen3 import (Qwen3ForCausalLM, Qwen3Spec, hf_tensor_shapes,
                                    load_checkpoint_tensors, num_parameters, rope_cache,
                                    write_random_checkpoint)
from kavor_amd.engine.scheduler import Scheduler
from kavor_amd.engine.sequence import Sequence
from kavor_amd.sampling_params import SamplingParams
from oracle import kvpath_oracle as ref

TINY = Qwen3Spec(vocab_size=512, hidden_size=256, intermediate_size=384, num_hidden_layers=2,
                 num_attention_heads=4, num_key_value_heads=2, head_dim=128,
                 max_position_embeddings=2048)


@pytest.fixture
def block_size(monkeypatch):
    monkeypatch.setattr(Sequence, "block_size", 64)
    return 64


def _scheduled_batches(bs, prompts, max_batched, num_blocks=64):
    """Yields (seqs, is_prefill) of successive steps with a fixed sampled token."""
    cfg = SimpleNamespace(max_num_seqs=8, max_num_batched_tokens=max_batched, eos=-1,
                          kvcache_block_size=bs, num_kvcache_blocks=num_blocks)
    sched = Scheduler(cfg)
    for p in prompts:
        sched.add(Sequence(p, SamplingParams(max_tokens=70, ignore_eos=True)))
    while not sched.is_finished():
        seqs, is_prefill = sched.schedule()
        yield seqs, is_prefill
        sched.postprocess(seqs, [7] * len(seqs), is_prefill)


def test_prefill_and_decode_metadata_match_oracle(block_size):
    rng = np.random.default_rng(0)
    shared = rng.integers(0, 500, 130).tolist()
    prompts = [shared + rng.integers(0, 500, n).tolist() for n in (5, 70, 400)]
    prompts.append(shared[:64] + [1, 2, 3])
    seen_prefix = seen_chunk = seen_decode = False
    for seqs, is_prefill in _scheduled_batches(block_size, prompts, max_batched=256):
        tables = [list(s.block_table) for s in seqs]
        if is_prefill:
            got = prefill_arrays(seqs, block_size)
            want = ref.prefill_metadata(tables, [s.num_cached_tokens for s in seqs],
                                        [s.num_scheduled_tokens for s in seqs], block_size)
            for key in ("slot_mapping", "positions", "cu_seqlens_q", "cu_seqlens_k"):
                assert got[key].tolist() == list(want[key]), key
            assert got["max_seqlen_q"] == want["max_seqlen_q"]
            assert got["max_seqlen_k"] == want["max_seqlen_k"]
            if want["block_tables"] is None:
                assert got["block_tables"] is None
            else:
                seen_prefix = True
                assert got["block_tables"].tolist() == want["block_tables"]
            ids = np.concatenate([np.asarray(s.token_ids[s.num_cached_tokens:
                                                         s.num_cached_tokens + s.num_scheduled_tokens])
                                  for s in seqs])
            assert got["input_ids"].tolist() == ids.tolist()
            seen_chunk |= any(s.num_cached_tokens + s.num_scheduled_tokens < s.num_tokens for s in seqs)
        else:
            seen_decode = True
            got = decode_arrays(seqs, block_size)
            want = ref.decode_metadata(tables, [len(s) for s in seqs], block_size)
            for key in ("slot_mapping", "positions", "context_lens"):
                assert got[key].tolist() == list(want[key]), key
            assert got["block_tables"].tolist() == want["block_tables"]
            assert got["input_ids"].tolist() == [s.last_token for s in seqs]
    assert seen_prefix and seen_chunk and seen_decode


def test_decode_staging_pads_rows(block_size):
    from kavor_amd.engine.metadata import DecodeStaging

    seqs = [Sequence(list(range(n)), SamplingParams(temperature=t)) for n, t in ((1, 0.0), (64, 0.75), (65, 1.5))]
    for i, s in enumerate(seqs):
        s.block_table = list(range(10 * i, 10 * i + s.num_blocks))
    st = DecodeStaging(rows=8, width=4, device="cpu", pin=False)
    st.fill(seqs, block_size, 4)
    m = st.views(4)
    assert m.temperatures.tolist() == [0.0, 0.75, 1.5, 0.0]
    assert m.context_lens.tolist() == [1, 64, 65, 0]
    assert m.slot_mapping.tolist() == [0, 10 * 64 + 63, 21 * 64 + 0, -1]
    assert m.positions.tolist() == [0, 63, 64, 0]
    assert m.block_tables[2, :2].tolist() == [20, 21]
    with pytest.raises(ValueError):
        st.fill(seqs, block_size, 2)



def test_decode_staging_refill_edges():
    """Refilling the same staging buffer: each row gets its table and a -1 after it when
    it is narrower than the buffer (columns past that keep stale entries, which the
    kernels never read); a table as wide as the buffer gets no -1; rows past the batch
    are padding; an empty batch pads every row; too few blocks or too many are refused."""
    from kavor_amd.engine.metadata import DecodeStaging

    bs = 64
    seqs = [Sequence(list(range(n)), SamplingParams()) for n in (200, 70, 256)]
    tables = [[5, 6, 7, 8], [9, 10], [11, 12, 13, 14]]
    for s, t in zip(seqs, tables):
        s.block_table = list(t)
    st = DecodeStaging(rows=4, width=4, device="cpu", pin=False)
    st.fill(seqs, bs, 4)
    assert st._htab[:3].tolist() == [[5, 6, 7, 8], [9, 10, -1, 0], [11, 12, 13, 14]]
    assert st.views(4).slot_mapping.tolist() == [8 * 64 + 7, 10 * 64 + 5, 14 * 64 + 63, -1]
    # the same rows now hold shorter tables: stale columns past the -1 stay as they were
    short = [Sequence(list(range(n)), SamplingParams()) for n in (3, 65)]
    short[0].block_table, short[1].block_table = [1], [2, 3]
    st.fill(short, bs, 3)
    assert st._htab[:3].tolist() == [[1, -1, 7, 8], [2, 3, -1, 0], [11, 12, 13, 14]]
    assert st.views(3).context_lens.tolist() == [3, 65, 0]
    assert st.views(3).input_ids.tolist() == [2, 64, 0]
    st.fill([], bs, 2)
    assert st.views(2).slot_mapping.tolist() == [-1, -1]
    assert st.views(2).context_lens.tolist() == [0, 0]
    bad = Sequence(list(range(130)), SamplingParams())
    bad.block_table = [1, 2]  # 2 pages of 64 hold 128 of 130 tokens
    with pytest.raises(ValueError, match="2 blocks for 130 tokens"):
        st.fill([bad], bs, 1)
    wide = Sequence(list(range(10)), SamplingParams())
    wide.block_table = [1, 2, 3, 4, 5]
    with pytest.raises(ValueError, match="table width 4"):
        st.fill([wide], bs, 1)

def test_page_pool_views_match_layout():
    model = Qwen3ForCausalLM(TINY, "cpu")
    pool = CachePool(model, TINY.num_key_value_heads, TINY.head_dim, block_size=64)
    assert pool.page_bytes == 2 * 64 * 2 * 128 * 2
    layout = pool.allocate(5, "cpu")
    assert layout.num_pools == TINY.num_hidden_layers
    for layer_idx, layer in enumerate(model.layers):
        kc, vc = layer.self_attn.attn.k_cache[0], layer.self_attn.attn.v_cache[0]
        wk, wv = ref.page_views(pool.pools[layer_idx], 64, 2, 128)
        assert kc.shape == wk.shape and kc.stride() == wk.stride() == (2 * 64 * 256, 256, 128, 1)
        assert kc.data_ptr() == wk.data_ptr() and vc.data_ptr() == wv.data_ptr()
    # a write through block 3's V view lands in the second half of page 3 of that layer
    model.layers[1].self_attn.attn.v_cache[0][3, 0, 0, 0] = 1.0
    page = pool.pools[1, 3].view(torch.bfloat16)
    assert page[64 * 256].item() == 1.0
    assert pool.blocks_for_budget(3 * layout.bytes_per_block + 1) == 3
    pool.copy_blocks([3], [4])
    assert torch.equal(pool.pools[:, 4], pool.pools[:, 3])


def test_product_rope_table_equals_oracle():
    from oracle.layers_oracle import rope_table

    assert torch.equal(rope_cache(128, 300, 1e6, "cpu"), rope_table(128, 300, 1e6))


def test_checkpoint_round_trip(tmp_path):
    path = write_random_checkpoint(tmp_path / "tiny", TINY, seed=3)
    assert Qwen3Spec.from_pretrained(path) == TINY
    tensors = load_checkpoint_tensors(path)
    assert {k: tuple(v.shape) for k, v in tensors.items()} == hf_tensor_shapes(TINY)
    assert sum(v.numel() for v in tensors.values()) == num_parameters(TINY)
    model = Qwen3ForCausalLM(TINY, "cpu")
    model.load_hf_state(tensors)
    a = model.layers[1].self_attn
    q = TINY.num_attention_heads * TINY.head_dim
    kv = TINY.num_key_value_heads * TINY.head_dim
    assert torch.equal(a.qkv_proj[q:q + kv], tensors["model.layers.1.self_attn.k_proj.weight"])
    assert torch.equal(model.layers[0].mlp.gate_up_proj[TINY.intermediate_size:],
                       tensors["model.layers.0.mlp.up_proj.weight"])
    assert model.lm_head is model.embed_tokens
    del tensors["model.layers.0.mlp.down_proj.weight"]
    with pytest.raises(KeyError, match="down_proj"):
        Qwen3ForCausalLM(TINY, "cpu").load_hf_state(tensors)


def test_qwen3_0_6b_spec_size():
    spec = Qwen3Spec.qwen3_0_6b()
    assert (spec.num_hidden_layers, spec.hidden_size, spec.num_attention_heads,
            spec.num_key_value_heads, spec.head_dim, spec.vocab_size) == (28, 1024, 16, 8, 128, 151936)
    assert num_parameters(spec) == 596_049_920


def test_config_rejects_multi_gpu_and_odd_pages():
    from kavor_amd.config import Config

    with pytest.raises(ValueError, match="one GPU"):
        Config(TINY, tensor_parallel_size=2)
    with pytest.raises(ValueError, match="multiple of 64"):
        Config(TINY, kvcache_block_size=100)
    assert Config(TINY, max_model_len=10**6).max_model_len == TINY.max_position_embeddings
