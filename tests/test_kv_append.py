"""GPU parity of the KV append (kvp_append_bf16 via kavor_amd.layers.attention.store_kvcache)
against the oracle: bit-exact, whole caches compared so untouched slots are checked too."""

import numpy as np
import pytest
import torch

from oracle import kvpath_oracle as ref
from tests.helpers import gen, randn_bf16, interleaved_pool, qkv_views, bits_equal
from tests.test_golden import load, bf16

pytestmark = pytest.mark.gpu


def _store(*args):
    from kavor_amd.layers.attention import store_kvcache

    store_kvcache(*args)


def _oracle_append(key, value, kc, vc, slots):
    kc, vc = kc.clone(), vc.clone()
    ref.kv_append(ref.bf16_bits(key), ref.bf16_bits(value), ref.bf16_bits(kc), ref.bf16_bits(vc),
                  slots.numpy())
    return kc, vc


@pytest.mark.parametrize("shuffle_pad", [False, True])
def test_append_full_size_contiguous(cuda_device, shuffle_pad):
    """4096 tokens x 8 kv heads x 128, caches [512, 256, 8, 128], 3968 distinct slots from a
    permutation of 131072 plus 128 padding slots (-1) at the tail or shuffled in."""
    g = gen(1000 + shuffle_pad)
    n, hkv, d, nb, bs = 4096, 8, 128, 512, 256
    key, value = randn_bf16((n, hkv, d), g), randn_bf16((n, hkv, d), g)
    kc, vc = randn_bf16((nb, bs, hkv, d), g), randn_bf16((nb, bs, hkv, d), g)
    slots = torch.cat([torch.randperm(nb * bs, generator=g)[:n - 128].to(torch.int32),
                       torch.full((128,), -1, dtype=torch.int32)])
    if shuffle_pad:
        slots = slots[torch.randperm(n, generator=g)]
    want_k, want_v = _oracle_append(key, value, kc, vc, slots)
    dk, dv = kc.to(cuda_device), vc.to(cuda_device)
    _store(key.to(cuda_device), value.to(cuda_device), dk, dv, slots.to(cuda_device))
    torch.cuda.synchronize()
    assert bits_equal(dk.cpu(), want_k)
    assert bits_equal(dv.cpu(), want_v)


@pytest.mark.parametrize("hkv,d,bs", [(8, 128, 256), (2, 128, 64), (1, 64, 16), (4, 256, 32), (3, 128, 8)])
def test_append_engine_page_layout(cuda_device, hkv, d, bs):
    """Kavor's interleaved pages (block stride = 2*bs*Hkv*D) with Qwen3 strides: k
    contiguous, v a view into the fused qkv output (row stride (Hq+2Hkv)*D)."""
    g = gen(2000 + hkv * d + bs)
    nb, n = 40, 300
    pool, kc, vc = interleaved_pool(nb, bs, hkv, d, g)
    _, key, value = qkv_views(n, 2 * hkv, hkv, d, g)
    assert value.stride(0) == 4 * hkv * d
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    slots[torch.randperm(n, generator=g)[:37]] = -1
    want_pool = pool.clone()
    wk, wv = ref.page_views(want_pool, bs, hkv, d)
    ref.kv_append(ref.bf16_bits(key), ref.bf16_bits(value), ref.bf16_bits(wk), ref.bf16_bits(wv), slots.numpy())
    dpool = pool.to(cuda_device)
    dk, dv = ref.page_views(dpool, bs, hkv, d)
    _store(key.to(cuda_device), value.to(cuda_device), dk, dv, slots.to(cuda_device))
    torch.cuda.synchronize()
    assert torch.equal(dpool.cpu(), want_pool)


def test_append_duplicate_slots_do_not_fault(cuda_device):
    """Graph capture appends with every slot 0 (model_runner.py:272, 301-308): no fault,
    every other slot untouched, and slot 0 holds source data: writers race per 16-byte
    vector, so each 16-byte chunk of slot 0 equals that chunk of one of the tokens."""
    g = gen(3)
    n, hkv, d, nb, bs = 64, 8, 128, 4, 256
    key, value = randn_bf16((n, hkv, d), g), randn_bf16((n, hkv, d), g)
    kc, vc = randn_bf16((nb, bs, hkv, d), g), randn_bf16((nb, bs, hkv, d), g)
    dk, dv = kc.to(cuda_device), vc.to(cuda_device)
    _store(key.to(cuda_device), value.to(cuda_device), dk, dv, torch.zeros(n, dtype=torch.int32, device=cuda_device))
    torch.cuda.synchronize()
    hk, hv = dk.cpu(), dv.cpu()
    assert bits_equal(hk.view(-1, hkv, d)[1:], kc.view(-1, hkv, d)[1:])
    assert bits_equal(hv.view(-1, hkv, d)[1:], vc.view(-1, hkv, d)[1:])
    for got, src in ((hk[0, 0], key), (hv[0, 0], value)):
        chunks = got.reshape(-1, 8).view(torch.int16)
        cand = src.reshape(n, -1, 8).view(torch.int16)
        for c in range(chunks.shape[0]):
            assert (cand[:, c] == chunks[c]).all(dim=-1).any(), f"chunk {c} matches no token"


def test_append_out_of_range_slots_are_skipped(cuda_device):
    """Slots outside the pool (other than -1) are skipped instead of written out of bounds."""
    g = gen(4)
    n, hkv, d, nb, bs = 8, 2, 128, 2, 64
    key, value = randn_bf16((n, hkv, d), g), randn_bf16((n, hkv, d), g)
    kc, vc = randn_bf16((nb, bs, hkv, d), g), randn_bf16((nb, bs, hkv, d), g)
    slots = torch.tensor([0, 127, 128, -5, 1 << 30, -1, 5, 64], dtype=torch.int32)
    keep = slots.clone()
    keep[(keep < 0) | (keep >= nb * bs)] = -1
    want_k, want_v = _oracle_append(key, value, kc, vc, keep)
    dk, dv = kc.to(cuda_device), vc.to(cuda_device)
    _store(key.to(cuda_device), value.to(cuda_device), dk, dv, slots.to(cuda_device))
    torch.cuda.synchronize()
    assert bits_equal(dk.cpu(), want_k) and bits_equal(dv.cpu(), want_v)


def test_append_token_permutation_is_bitwise_invariant(cuda_device):
    g = gen(5)
    n, hkv, d, nb, bs = 512, 8, 128, 16, 256
    key, value = randn_bf16((n, hkv, d), g), randn_bf16((n, hkv, d), g)
    kc, vc = randn_bf16((nb, bs, hkv, d), g), randn_bf16((nb, bs, hkv, d), g)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    perm = torch.randperm(n, generator=g)
    outs = []
    for idx in (torch.arange(n), perm):
        dk, dv = kc.to(cuda_device), vc.to(cuda_device)
        _store(key[idx].to(cuda_device), value[idx].to(cuda_device), dk, dv, slots[idx].to(cuda_device))
        outs.append((dk.cpu(), dv.cpu()))
    assert bits_equal(outs[0][0], outs[1][0]) and bits_equal(outs[0][1], outs[1][1])


def test_append_graph_replay_matches_eager(cuda_device):
    """Capture once, then rewrite the slot buffer and replay: each replay equals the eager
    append with the same slots, bit for bit."""
    g = gen(6)
    n, hkv, d, nb, bs = 128, 8, 128, 8, 256
    key, value = randn_bf16((n, hkv, d), g).to(cuda_device), randn_bf16((n, hkv, d), g).to(cuda_device)
    base_k, base_v = randn_bf16((nb, bs, hkv, d), g).to(cuda_device), randn_bf16((nb, bs, hkv, d), g).to(cuda_device)
    kc, vc = base_k.clone(), base_v.clone()
    slots = torch.full((n,), -1, dtype=torch.int32, device=cuda_device)
    _store(key, value, kc, vc, slots)  # warm-up outside capture
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _store(key, value, kc, vc, slots)
    for step in range(3):
        new = torch.randperm(nb * bs, generator=gen(60 + step))[:n].to(torch.int32)
        new[:step * 7] = -1
        kc.copy_(base_k)
        vc.copy_(base_v)
        slots.copy_(new.to(cuda_device))
        graph.replay()
        torch.cuda.synchronize()
        rk, rv = kc.clone(), vc.clone()
        kc.copy_(base_k)
        vc.copy_(base_v)
        _store(key, value, kc, vc, new.to(cuda_device))
        torch.cuda.synchronize()
        assert bits_equal(rk, kc) and bits_equal(rv, vc)


def test_append_empty_batch(cuda_device):
    kc = torch.zeros(2, 64, 2, 128, dtype=torch.bfloat16, device=cuda_device)
    e = torch.empty(0, 2, 128, dtype=torch.bfloat16, device=cuda_device)
    _store(e, e, kc, kc.clone(), torch.empty(0, dtype=torch.int32, device=cuda_device))
    torch.cuda.synchronize()
    assert torch.count_nonzero(kc) == 0


def test_append_golden(cuda_device):
    f = load("append_small")
    nb, bs, hkv, d = (int(x) for x in f["dims"])
    pool = torch.from_numpy(f["pool_before"].copy()).to(cuda_device)
    kc, vc = ref.page_views(pool, bs, hkv, d)
    n = f["key"].shape[0]
    key = bf16(f["key"]).to(cuda_device)
    wide = torch.zeros(n, 4 * hkv * d, dtype=torch.bfloat16, device=cuda_device)
    wide[:, 3 * hkv * d:] = bf16(f["value"]).reshape(n, -1).to(cuda_device)
    value = wide[:, 3 * hkv * d:].view(n, hkv, d)
    _store(key, value, kc, vc, torch.from_numpy(f["slot_mapping"]).to(cuda_device))
    torch.cuda.synchronize()
    assert np.array_equal(pool.cpu().numpy(), f["pool_after"])


@pytest.mark.parametrize("n,hkv,d", [(1, 8, 128), (3, 8, 128), (13, 2, 64), (9, 16, 256), (5, 12, 128)])
def test_append_ragged_counts_and_long_rows(cuda_device, n, hkv, d):
    """Token counts that leave a wave with one token and a workgroup partly empty, and
    rows longer than one pass of the wave (16 x 256 bf16 = 512 chunks per row)."""
    g = gen(3000 + n * hkv + d)
    nb, bs = 6, 64
    key, value = randn_bf16((n, hkv, d), g), randn_bf16((n, hkv, d), g)
    kc, vc = randn_bf16((nb, bs, hkv, d), g), randn_bf16((nb, bs, hkv, d), g)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    if n > 2:
        slots[n // 2] = -1
    want_k, want_v = _oracle_append(key, value, kc, vc, slots)
    dk, dv = kc.to(cuda_device), vc.to(cuda_device)
    _store(key.to(cuda_device), value.to(cuda_device), dk, dv, slots.to(cuda_device))
    torch.cuda.synchronize()
    assert bits_equal(dk.cpu(), want_k) and bits_equal(dv.cpu(), want_v)
