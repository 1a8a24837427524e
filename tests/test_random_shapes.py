"""Seeded random shapes for the three path kernels against the oracle: GQA ratios 1, 2,
4, 5 and 8, block sizes 64-512, both page layouts, context and prefix lengths from a
single token to several pages, causal and not.  Each case prints its seed and shape
before it runs.  KVP_RANDOM_CASES sets the number of cases per kernel (default 12)."""

import math
import os

import pytest
import torch

from oracle import kvpath_oracle as ref
from tests.helpers import TOL, gen, randn_bf16, interleaved_pool, contiguous_caches, random_block_tables

pytestmark = pytest.mark.gpu
CASES = int(os.environ.get("KVP_RANDOM_CASES", "12"))
D = 128


def _shape(seed):
    g = gen(9000 + seed)
    pick = lambda xs: xs[int(torch.randint(0, len(xs), (1,), generator=g))]
    G = pick([1, 2, 4, 5, 8])
    hkv = pick([1, 2, 4, 8]) if G != 8 else pick([1, 2])
    bs = pick([64, 128, 256, 512])
    layout = pick(["contiguous", "interleaved"])
    return g, G, hkv, bs, layout


def _pool(g, nb, bs, hkv, layout):
    if layout == "contiguous":
        return contiguous_caches(nb, bs, hkv, D, g)
    _, kc, vc = interleaved_pool(nb, bs, hkv, D, g)
    return kc, vc


@pytest.mark.parametrize("seed", range(CASES))
def test_random_decode(cuda_device, seed):
    from kavor_amd.layers.attention import paged_decode

    g, G, hkv, bs, layout = _shape(seed)
    B = int(torch.randint(1, 70, (1,), generator=g))
    hi = int(torch.randint(1, 6000, (1,), generator=g))
    ctx = torch.randint(0, hi + 1, (B,), generator=g, dtype=torch.int32)
    print(f"decode seed={seed} B={B} G={G} hkv={hkv} bs={bs} {layout} ctx<= {hi}", flush=True)
    nb = sum(math.ceil(int(c) / bs) for c in ctx) + 2
    kc, vc = _pool(g, nb, bs, hkv, layout)
    bt = random_block_tables([int(c) for c in ctx], bs, nb, g)
    q = randn_bf16((B, G * hkv, D), g)
    d = cuda_device
    out = paged_decode(q.to(d), kc.to(d), vc.to(d), cache_seqlens=ctx.to(d), block_table=bt.to(d),
                       softmax_scale=D ** -0.5)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().float(), ref.paged_decode(q, kc, vc, bt, ctx, D ** -0.5), **TOL)


@pytest.mark.parametrize("seed", range(CASES))
def test_random_prefill(cuda_device, seed):
    from kavor_amd.layers.attention import varlen_prefill

    g, G, hkv, bs, layout = _shape(seed)
    nseq = int(torch.randint(1, 12, (1,), generator=g))
    qlens = [int(x) for x in torch.randint(1, 400, (nseq,), generator=g)]
    paged = bool(torch.randint(0, 2, (1,), generator=g))
    causal = bool(torch.randint(0, 4, (1,), generator=g))  # mostly causal, as the engine runs it
    prefix = [int(x) for x in torch.randint(0, 900, (nseq,), generator=g)] if paged else [0] * nseq
    klens = [a + b for a, b in zip(qlens, prefix)]
    max_q = max(qlens) if bool(torch.randint(0, 3, (1,), generator=g)) else max(1, max(qlens) // 3)
    print(f"prefill seed={seed} G={G} hkv={hkv} bs={bs} {layout} paged={paged} causal={causal} "
          f"qlens={qlens} prefix={prefix} max_q={max_q}", flush=True)
    q = randn_bf16((sum(qlens), G * hkv, D), g)
    cq = torch.tensor([0] + list(torch.tensor(qlens).cumsum(0)), dtype=torch.int32)
    ck = torch.tensor([0] + list(torch.tensor(klens).cumsum(0)), dtype=torch.int32)
    d = cuda_device
    if paged:
        nb = sum(math.ceil(k / bs) for k in klens) + 2
        kc, vc = _pool(g, nb, bs, hkv, layout)
        bt = random_block_tables(klens, bs, nb, g)
        if bool(torch.randint(0, 2, (1,), generator=g)):
            # prefix-cache hits: some sequences start with the full leading pages of an
            # earlier one (the plan ranks sequences that share a first block together)
            for s2 in range(1, nseq):
                s1 = int(torch.randint(0, s2 + 1, (1,), generator=g))
                m = min(prefix[s1], prefix[s2]) // bs
                if s1 != s2 and m:
                    bt[s2, :m] = bt[s1, :m]
        out = varlen_prefill(q.to(d), kc.to(d), vc.to(d), max_seqlen_q=max_q, cu_seqlens_q=cq.to(d),
                             max_seqlen_k=max(klens), cu_seqlens_k=ck.to(d), softmax_scale=D ** -0.5,
                             causal=causal, block_table=bt.to(d))
        want = ref.varlen_prefill(q, kc, vc, cq, ck, D ** -0.5, block_tables=bt, causal=causal)
    else:
        k = randn_bf16((sum(klens), hkv, D), g)
        v = randn_bf16((sum(klens), hkv, D), g)
        out = varlen_prefill(q.to(d), k.to(d), v.to(d), max_seqlen_q=max_q, cu_seqlens_q=cq.to(d),
                             max_seqlen_k=max(klens), cu_seqlens_k=ck.to(d), softmax_scale=D ** -0.5,
                             causal=causal)
        want = ref.varlen_prefill(q, k, v, cq, ck, D ** -0.5, causal=causal)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().float(), want, **TOL)


@pytest.mark.parametrize("seed", range(CASES))
def test_random_append(cuda_device, seed):
    from kavor_amd.layers.attention import store_kvcache

    g, _, hkv, bs, layout = _shape(seed)
    nb = int(torch.randint(2, 40, (1,), generator=g))
    n = min(int(torch.randint(1, 600, (1,), generator=g)), nb * bs)
    print(f"append seed={seed} n={n} hkv={hkv} bs={bs} {layout} blocks={nb}", flush=True)
    kc, vc = _pool(g, nb, bs, hkv, layout)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    slots[torch.rand(n, generator=g) < 0.1] = -1
    k = randn_bf16((n, hkv, D), g)
    v = randn_bf16((n, hkv, D), g)
    want_k, want_v = kc.clone(), vc.clone()
    ref.kv_append(ref.bf16_bits(k), ref.bf16_bits(v), ref.bf16_bits(want_k), ref.bf16_bits(want_v), slots.numpy())
    d = cuda_device
    kd, vd = kc.to(d), vc.to(d)
    store_kvcache(k.to(d), v.to(d), kd, vd, slots.to(d))
    torch.cuda.synchronize()
    assert torch.equal(kd.cpu().view(torch.int16), want_k.view(torch.int16))
    assert torch.equal(vd.cpu().view(torch.int16), want_v.view(torch.int16))
