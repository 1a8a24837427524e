"""The drop-in Attention module end to end on the GPU, driven through the Context exactly
as ModelRunner drives it (model_runner.py:385-473): a dense prefill that appends the
prompt, a prefix-cached (paged) prefill, then decode steps; each checked against the
oracle applied to the same page pool."""

import math

import pytest
import torch

from oracle import kvpath_oracle as ref
from tests.helpers import TOL, gen, randn_bf16, interleaved_pool, qkv_views

pytestmark = pytest.mark.gpu
BS, HQ, HKV, D = 256, 16, 8, 128
SCALE = D ** -0.5


def _i32(x, dev):
    return torch.tensor(x, dtype=torch.int32, device=dev)


def test_attention_prefill_prefix_decode(cuda_device):
    from kavor_amd.layers.attention import Attention
    from kavor_amd.utils.context import set_context, reset_context

    dev = cuda_device
    g = gen(300)
    nb = 40
    pool, kc, vc = interleaved_pool(nb, BS, HKV, D, g)
    pool = pool.to(dev)
    attn = Attention(HQ, D, SCALE, HKV)
    attn.k_cache[0], attn.v_cache[0] = ref.page_views(pool, BS, HKV, D)

    # three sequences with their block tables (block manager output)
    tables = [[3, 17, 9], [22], [5, 30, 31, 2]]
    lens = [600, 100, 800]

    # ---- dense prefill of the whole prompts (no prefix hits: block_tables None)
    meta = ref.prefill_metadata(tables, [0, 0, 0], lens, BS)
    T = sum(lens)
    q, k, v = qkv_views(T, HQ, HKV, D, g)
    set_context(True, _i32(meta["cu_seqlens_q"], dev), _i32(meta["cu_seqlens_k"], dev),
                meta["max_seqlen_q"], meta["max_seqlen_k"], _i32(meta["slot_mapping"], dev))
    out = attn(q.to(dev), k.to(dev), v.to(dev))
    torch.cuda.synchronize()
    reset_context()
    cu = torch.tensor(meta["cu_seqlens_q"])
    torch.testing.assert_close(out.cpu().float(), ref.varlen_prefill(q, k, v, cu, cu, SCALE), **TOL)
    # the prompt K/V now sit in the pages
    host_pool = pool.cpu()
    hk, hv = ref.page_views(host_pool, BS, HKV, D)
    want_k, want_v = kc.clone(), vc.clone()
    ref.kv_append(ref.bf16_bits(k), ref.bf16_bits(v), ref.bf16_bits(want_k), ref.bf16_bits(want_v),
                  meta["slot_mapping"])
    assert torch.equal(hk.contiguous().view(torch.int16), want_k.contiguous().view(torch.int16))
    assert torch.equal(hv.contiguous().view(torch.int16), want_v.contiguous().view(torch.int16))

    # ---- prefix-cached prefill: sequence 3 shares sequence 0's first two blocks
    tables.append([3, 17, 11])
    cached, new = 512, 150
    meta2 = ref.prefill_metadata([tables[3]], [cached], [new], BS)
    assert meta2["block_tables"] is not None
    q2, k2, v2 = qkv_views(new, HQ, HKV, D, g)
    set_context(True, _i32(meta2["cu_seqlens_q"], dev), _i32(meta2["cu_seqlens_k"], dev),
                meta2["max_seqlen_q"], meta2["max_seqlen_k"], _i32(meta2["slot_mapping"], dev),
                None, _i32(meta2["block_tables"], dev))
    out2 = attn(q2.to(dev), k2.to(dev), v2.to(dev))
    torch.cuda.synchronize()
    reset_context()
    host_pool = pool.cpu()
    hk, hv = ref.page_views(host_pool, BS, HKV, D)
    want2 = ref.varlen_prefill(q2, hk, hv, torch.tensor(meta2["cu_seqlens_q"]),
                               torch.tensor(meta2["cu_seqlens_k"]), SCALE,
                               block_tables=torch.tensor(meta2["block_tables"]))
    torch.testing.assert_close(out2.cpu().float(), want2, **TOL)
    # the prefix the new tokens attended to is sequence 0's prompt
    assert torch.equal(hk[3].view(torch.int16), want_k[3].view(torch.int16))
    lens.append(cached + new)

    # ---- two decode steps for all four sequences
    for step in range(2):
        lens = [n + 1 for n in lens]
        for i, n in enumerate(lens):
            if math.ceil(n / BS) > len(tables[i]):
                tables[i].append(35 + i)
        meta3 = ref.decode_metadata(tables, lens, BS)
        B = len(lens)
        q3, k3, v3 = qkv_views(B, HQ, HKV, D, g)
        set_context(False, slot_mapping=_i32(meta3["slot_mapping"], dev),
                    context_lens=_i32(meta3["context_lens"], dev),
                    block_tables=_i32(meta3["block_tables"], dev))
        out3 = attn(q3.to(dev), k3.to(dev), v3.to(dev))
        torch.cuda.synchronize()
        reset_context()
        assert out3.shape == (B, 1, HQ, D)
        host_pool = pool.cpu()
        hk, hv = ref.page_views(host_pool, BS, HKV, D)
        want3 = ref.paged_decode(q3, hk, hv, torch.tensor(meta3["block_tables"]),
                                 torch.tensor(meta3["context_lens"]), SCALE)
        torch.testing.assert_close(out3[:, 0].cpu().float(), want3, **TOL)
        # the decoded token's K row was appended before attention read it
        for i in range(B):
            s = meta3["slot_mapping"][i]
            assert torch.equal(hk[s // BS, s % BS].view(torch.int16), k3[i].view(torch.int16))
