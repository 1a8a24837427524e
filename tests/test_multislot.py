"""Attention modules with several KV slots (num_kv_slots > 1).

The reference binds one page pool per (module, slot) (kavor/engine/cache_pool.py:311-322),
and its Attention reads k_cache[slot] / v_cache[slot] (flash_attention_kvcache.py:68-72);
Ouro runs its shared layers once per loop step, each step with its own slot
(kavor/models/ouro.py:179-185).  The CPU test checks the binding; the GPU test drives
forward(q, k, v, slot=1) through a prefill, a prefix-cached prefill and a decode step and
checks that slot 1's pages receive the appends and are the ones attended over, while
slot 0's pool (and the other module's) keeps every byte.
"""

import pytest
import torch
from torch import nn

from kavor_amd.engine.cache_pool import CachePool
from kavor_amd.layers.attention import Attention
from oracle import kvpath_oracle as ref
from tests.helpers import TOL, gen, randn_bf16

BS, HQ, HKV, D = 64, 8, 4, 128
SCALE = D ** -0.5


class _Looped(nn.Module):
    """A shared attention layer run in two loop steps (two KV slots), then a plain one."""

    def __init__(self):
        super().__init__()
        self.shared = Attention(HQ, D, SCALE, HKV, num_kv_slots=2)
        self.last = Attention(HQ, D, SCALE, HKV)


def _pool(device, nb=12):
    model = _Looped()
    pool = CachePool(model, HKV, D, BS)
    pool.allocate(nb, device)
    return model, pool


def test_two_slots_bind_two_pools():
    model, pool = _pool("cpu")
    layout = pool.layout
    assert layout.num_pools == 3 and [s for _, s in pool.slots] == [0, 1, 0]
    assert [m for m, _ in pool.slots] == [model.shared, model.shared, model.last]
    page_elems = layout.page_bytes // 2
    for i, (module, slot) in enumerate(pool.slots):
        kc, vc = module.k_cache[slot], module.v_cache[slot]
        assert kc.shape == (12, BS, HKV, D) and kc.stride() == (page_elems, HKV * D, D, 1)
        base = pool.pools[i].data_ptr()
        assert kc.data_ptr() == base and vc.data_ptr() == base + BS * HKV * D * 2
        # the views are exactly the oracle's restatement of the page layout
        rk, rv = ref.page_views(pool.pools[i], BS, HKV, D)
        assert rk.data_ptr() == kc.data_ptr() and rk.stride() == kc.stride()
        assert rv.data_ptr() == vc.data_ptr()
    # a write through slot 1's view lands in pool 1 only
    pool.pools.zero_()
    model.shared.k_cache[1][3, 5, 2] = torch.ones(D, dtype=torch.bfloat16)
    touched = [bool(pool.pools[i].any()) for i in range(3)]
    assert touched == [False, True, False]
    pool.release()
    assert model.shared.k_cache[1].numel() == 0 and model.last.k_cache[0].numel() == 0


def _i32(x, dev):
    return torch.tensor(x, dtype=torch.int32, device=dev)


@pytest.mark.gpu
def test_forward_on_slot_1_uses_only_slot_1(cuda_device):
    from kavor_amd.utils.context import reset_context, set_context

    dev = cuda_device
    g = gen(700)
    model, pool = _pool(dev)
    pool.pools.copy_(torch.randint(0, 256, pool.pools.shape, generator=g, dtype=torch.uint8).to(dev))
    # finite bf16 everywhere: clear each element's exponent top bit (no Inf / NaN patterns)
    pool.pools.view(torch.int16).bitwise_and_(~0x4000)
    before = pool.pools.clone()
    attn = model.shared
    kc1, vc1 = attn.k_cache[1], attn.v_cache[1]

    # ---- prefill of two prompts through slot 1 (dense: no prefix), appending into slot 1
    tables, lens = [[4, 9, 1], [7]], [150, 40]
    meta = ref.prefill_metadata(tables, [0, 0], lens, BS)
    T = sum(lens)
    q, k, v = randn_bf16((T, HQ, D), g), randn_bf16((T, HKV, D), g), randn_bf16((T, HKV, D), g)
    set_context(True, _i32(meta["cu_seqlens_q"], dev), _i32(meta["cu_seqlens_k"], dev),
                meta["max_seqlen_q"], meta["max_seqlen_k"], _i32(meta["slot_mapping"], dev))
    out = attn(q.to(dev), k.to(dev), v.to(dev), slot=1)
    torch.cuda.synchronize()
    reset_context()
    cu = torch.tensor(meta["cu_seqlens_q"])
    torch.testing.assert_close(out.cpu().float(), ref.varlen_prefill(q, k, v, cu, cu, SCALE), **TOL)
    want_k, want_v = ref.page_views(before[1].cpu(), BS, HKV, D)
    want_k, want_v = want_k.clone(), want_v.clone()
    ref.kv_append(ref.bf16_bits(k), ref.bf16_bits(v), ref.bf16_bits(want_k), ref.bf16_bits(want_v),
                  meta["slot_mapping"])

    # ---- prefix-cached prefill through slot 1: a third sequence reuses sequence 0's first
    # two pages (128 tokens) and appends 30 new tokens; attention reads slot 1's pages
    tables3, cached, n3 = [[4, 9, 2]], [128], [30]
    meta3 = ref.prefill_metadata(tables3, cached, n3, BS)
    q3, k3, v3 = randn_bf16((30, HQ, D), g), randn_bf16((30, HKV, D), g), randn_bf16((30, HKV, D), g)
    bt3 = _i32(ref.pad_block_tables(tables3), dev)
    set_context(True, _i32(meta3["cu_seqlens_q"], dev), _i32(meta3["cu_seqlens_k"], dev),
                meta3["max_seqlen_q"], meta3["max_seqlen_k"], _i32(meta3["slot_mapping"], dev),
                block_tables=bt3)
    out3 = attn(q3.to(dev), k3.to(dev), v3.to(dev), slot=1)
    torch.cuda.synchronize()
    reset_context()
    ref.kv_append(ref.bf16_bits(k3), ref.bf16_bits(v3), ref.bf16_bits(want_k), ref.bf16_bits(want_v),
                  meta3["slot_mapping"])
    want3 = ref.varlen_prefill(q3, want_k, want_v, torch.tensor(meta3["cu_seqlens_q"]),
                               torch.tensor(meta3["cu_seqlens_k"]), SCALE, block_tables=bt3.cpu())
    torch.testing.assert_close(out3.cpu().float(), want3, **TOL)

    # ---- one decode step through slot 1 for the three sequences
    all_tables, seq_lens = [[4, 9, 1], [7], [4, 9, 2]], [151, 41, 159]
    dmeta = ref.decode_metadata(all_tables, seq_lens, BS)
    qd, kd, vd = randn_bf16((3, HQ, D), g), randn_bf16((3, HKV, D), g), randn_bf16((3, HKV, D), g)
    bt = _i32(ref.pad_block_tables(all_tables), dev)
    ctx = _i32(dmeta["context_lens"], dev)
    set_context(False, slot_mapping=_i32(dmeta["slot_mapping"], dev), context_lens=ctx, block_tables=bt)
    outd = attn(qd.to(dev), kd.to(dev), vd.to(dev), slot=1)
    torch.cuda.synchronize()
    reset_context()
    ref.kv_append(ref.bf16_bits(kd), ref.bf16_bits(vd), ref.bf16_bits(want_k), ref.bf16_bits(want_v),
                  dmeta["slot_mapping"])
    wantd = ref.paged_decode(qd, want_k, want_v, bt.cpu(), ctx.cpu(), SCALE)
    torch.testing.assert_close(outd.reshape(3, HQ, D).cpu().float(), wantd, **TOL)

    # slot 1's pages hold exactly the appended rows; slot 0's pool and the other
    # module's pool keep every byte
    assert torch.equal(kc1.cpu().contiguous().view(torch.int16), want_k.contiguous().view(torch.int16))
    assert torch.equal(vc1.cpu().contiguous().view(torch.int16), want_v.contiguous().view(torch.int16))
    assert torch.equal(pool.pools[0], before[0]) and torch.equal(pool.pools[2], before[2])
    pool.release()
