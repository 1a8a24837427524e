"""The one-launch decode step (kvp_paged_decode_fused_bf16): q/k RMSNorm + RoPE of each
sequence's new token from its qkv row, the append of its k / v, and paged decode attention.

It is checked against the same step done by separate launches (the fused q/k norm + RoPE
+ append kernel, then paged decode) on identical inputs and page pools: after the call
both pools must be identical byte for byte (the rotated k and the raw v at each slot,
nothing else touched), and the attention output must match the fp32 oracle over the
appended caches within atol 2e-2 / rtol 1e-2.  The new token is the last of its context
and is folded in from registers rather than read back, so the cases cover contexts of
one token, a new token that opens a page, contexts split across several work ranges,
padding rows (context 0, slot -1) and a position outside the RoPE table; the slots being
appended hold NaN before the call, as recycled page memory may.
"""

import math

import pytest
import torch

from kavor_amd.layers.attention import paged_decode, paged_decode_fused
from kavor_amd.layers.fused import qk_norm_rope_append
from oracle import kvpath_oracle as ref
from oracle import layers_oracle as lref
from tests.helpers import TOL, gen, interleaved_pool, random_block_tables, randn_bf16

pytestmark = pytest.mark.gpu
D, EPS = 128, 1e-6


def _case(dev, seed, hq, hkv, bs, ctxs, pad=0, max_pos=40960):
    g = gen(seed)
    B = len(ctxs) + pad
    nb = sum(math.ceil(c / bs) for c in ctxs) + 3
    pool, _, _ = interleaved_pool(nb, bs, hkv, D, g)
    bt = random_block_tables(list(ctxs) + [1] * pad, bs, nb, g)
    ctx = torch.tensor(list(ctxs) + [0] * pad, dtype=torch.int32)
    pos = (ctx - 1).clamp(min=0)
    slots = torch.full((B,), -1, dtype=torch.int32)
    for b, c in enumerate(ctxs):
        t = c - 1
        slots[b] = int(bt[b, t // bs]) * bs + t % bs
    qkv = randn_bf16((B, (hq + 2 * hkv) * D), g)
    qw, kw = randn_bf16((D,), g, 0.5) + 1, randn_bf16((D,), g, 0.5) + 1
    table = lref.rope_table(D, max_pos, 1e6)
    host = dict(pool=pool, bt=bt, ctx=ctx, pos=pos, slots=slots, qkv=qkv, qw=qw, kw=kw, table=table)
    return host, {k: v.to(dev) for k, v in host.items()}


def _separate(d, hq, hkv, bs):
    kc, vc = ref.page_views(d["pool"], bs, hkv, D)
    q = qk_norm_rope_append(d["qkv"], d["pos"], d["table"], d["qw"], d["kw"], EPS, hq, hkv, kc, vc, d["slots"])
    return paged_decode(q, kc, vc, d["ctx"], d["bt"], D ** -0.5)


def _fused(d, hq, hkv, bs):
    kc, vc = ref.page_views(d["pool"], bs, hkv, D)
    return paged_decode_fused(d["qkv"], d["table"], d["qw"], d["kw"], EPS, hq, hkv, kc, vc,
                              d["slots"], d["ctx"], d["bt"], D ** -0.5)


@pytest.mark.parametrize("G,hkv,bs", [(1, 2, 64), (2, 8, 256), (4, 8, 256), (5, 8, 256), (8, 2, 128)])
def test_fused_decode_equals_separate_launches(cuda_device, G, hkv, bs):
    hq = G * hkv
    ctxs = [1, 2, bs, bs + 1, 3 * bs - 1, 1500, 4000, 777]
    host, d1 = _case(cuda_device, 100 + G, hq, hkv, bs, ctxs, pad=3)
    d2 = {k: v.clone() for k, v in d1.items()}
    # the slots the step appends hold NaN beforehand: nothing may read them before the
    # append (a masked row times a NaN would still be NaN)
    kc2, vc2 = ref.page_views(d2["pool"], bs, hkv, D)
    for slot in host["slots"].tolist():
        if slot >= 0:
            kc2[slot // bs, slot % bs] = float("nan")
            vc2[slot // bs, slot % bs] = float("nan")
    o_sep = _separate(d1, hq, hkv, bs)
    o_fused = _fused(d2, hq, hkv, bs)
    torch.cuda.synchronize()
    # the append is the same bytes, and nothing else in the pool moved
    assert torch.equal(d1["pool"].cpu(), d2["pool"].cpu())
    assert not torch.equal(d2["pool"].cpu(), host["pool"])
    # attention over the appended caches, fp32 oracle
    kc, vc = ref.page_views(d2["pool"].cpu(), bs, hkv, D)
    wq, _, _ = lref.qk_norm_rope(host["qkv"], host["pos"], host["table"], host["qw"], host["kw"], EPS, hq, hkv)
    want = ref.paged_decode(wq, kc, vc, host["bt"], host["ctx"], D ** -0.5)
    got = o_fused.cpu()
    torch.testing.assert_close(got.float(), want, **TOL)
    torch.testing.assert_close(got.float(), o_sep.cpu().float(), **TOL)
    assert torch.count_nonzero(got[len(ctxs):]) == 0  # padding rows: zeros


def test_fused_decode_position_outside_table_poisons_the_row(cuda_device):
    hq, hkv, bs = 16, 8, 256
    # the decode token of the 1001-token context sits at position 1000, outside the table
    host, d = _case(cuda_device, 7, hq, hkv, bs, [300, 1001, 900], max_pos=1000)
    o = _fused(d, hq, hkv, bs).cpu()
    assert torch.isnan(o[1].float()).all()
    assert torch.isfinite(o[[0, 2]].float()).all()


def test_fused_decode_replays_in_a_graph(cuda_device):
    """Captured once with one batch's metadata, replayed with another's (new contexts,
    slots and qkv rows written into the same buffers): every replay equals an
    eager call on a copy of the pool."""
    hq, hkv, bs = 16, 8, 256
    host, d = _case(cuda_device, 8, hq, hkv, bs, [500, 1200, 64, 2000])
    kc, vc = ref.page_views(d["pool"], bs, hkv, D)
    out = torch.empty(4, hq, D, dtype=torch.bfloat16, device=cuda_device)

    def call():
        paged_decode_fused(d["qkv"], d["table"], d["qw"], d["kw"], EPS, hq, hkv, kc, vc,
                           d["slots"], d["ctx"], d["bt"], D ** -0.5, out=out)

    call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    # contexts with the same page counts as the captured batch (2, 5, 1 and 8 pages)
    for step, ctxs in enumerate(([480, 1190, 60, 1990], [470, 1100, 30, 1800], [510, 1210, 64, 2010])):
        h2, d2 = _case(cuda_device, 20 + step, hq, hkv, bs, ctxs)
        assert d2["pool"].shape == d["pool"].shape and d2["bt"].shape == d["bt"].shape
        for k in ("bt", "ctx", "slots", "qkv", "qw", "kw"):
            d[k].copy_(d2[k])
        d["pool"].copy_(d2["pool"])
        eager = _fused(d2, hq, hkv, bs)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.cpu().view(torch.int16), eager.cpu().view(torch.int16))
        assert torch.equal(d["pool"].cpu(), d2["pool"].cpu())


@pytest.mark.parametrize("seed", range(int(__import__("os").environ.get("KVP_RANDOM_CASES", "12"))))
def test_fused_decode_random_shapes(cuda_device, seed):
    """Seeded random batches (GQA 1, 2, 4, 5 or 8, block sizes 64-512, contexts from one
    token to several pages, padding rows): the pools equal the separate launches' byte
    for byte and the output matches the oracle."""
    g = gen(7000 + seed)
    pick = lambda xs: xs[int(torch.randint(0, len(xs), (1,), generator=g))]
    G, bs = pick([1, 2, 4, 5, 8]), pick([64, 128, 256, 512])
    hkv = pick([1, 2, 4, 8]) if G != 8 else pick([1, 2])
    hq = G * hkv
    B = int(torch.randint(1, 40, (1,), generator=g))
    hi = int(torch.randint(1, 5000, (1,), generator=g))
    ctxs = [int(x) for x in torch.randint(1, hi + 1, (B,), generator=g)]
    pad = int(torch.randint(0, 3, (1,), generator=g))
    print(f"fused decode seed={seed} G={G} hkv={hkv} bs={bs} B={B} pad={pad} ctx<= {hi}", flush=True)
    host, d1 = _case(cuda_device, 7100 + seed, hq, hkv, bs, ctxs, pad=pad)
    d2 = {k: v.clone() for k, v in d1.items()}
    o_sep = _separate(d1, hq, hkv, bs)
    o_fused = _fused(d2, hq, hkv, bs)
    torch.cuda.synchronize()
    assert torch.equal(d1["pool"].cpu(), d2["pool"].cpu())
    kc, vc = ref.page_views(d2["pool"].cpu(), bs, hkv, D)
    wq, _, _ = lref.qk_norm_rope(host["qkv"], host["pos"], host["table"], host["qw"], host["kw"], EPS, hq, hkv)
    want = ref.paged_decode(wq, kc, vc, host["bt"], host["ctx"], D ** -0.5)
    torch.testing.assert_close(o_fused.cpu().float(), want, **TOL)
    torch.testing.assert_close(o_fused.cpu().float(), o_sep.cpu().float(), **TOL)
