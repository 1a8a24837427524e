"""GPU parity of varlen prefill (kvp_varlen_prefill_bf16 via kavor_amd.layers.attention.varlen_prefill)
against the fp32 oracle, within atol 2e-2 / rtol 1e-2 on the bf16 output."""

import math

import numpy as np
import pytest
import torch

from oracle import kvpath_oracle as ref
from tests.helpers import (TOL, gen, randn_bf16, interleaved_pool, contiguous_caches, random_block_tables,
                           bits_equal, relocate_pages)
from tests.test_golden import load, bf16

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def _prefill(q, k, v, cq, ck, max_q, scale=SCALE, causal=True, bt=None):
    from kavor_amd.layers.attention import varlen_prefill

    return varlen_prefill(q, k, v, max_seqlen_q=max_q, cu_seqlens_q=cq, max_seqlen_k=0,
                          cu_seqlens_k=ck, softmax_scale=scale, causal=causal, block_table=bt)


def _cu(lens):
    return torch.tensor(np.cumsum([0] + list(lens)), dtype=torch.int32)


def _dense_case(seed, qlens, hq, hkv, qkv_view=True):
    g = gen(seed)
    T = sum(qlens)
    q = randn_bf16((T, hq, 128), g)
    if qkv_view:  # Qwen3: k fresh, v a view into the fused projection
        wide = randn_bf16((T, (hq + 2 * hkv) * 128), g)
        v = wide[:, (hq + hkv) * 128:].view(T, hkv, 128)
    else:
        v = randn_bf16((T, hkv, 128), g)
    k = randn_bf16((T, hkv, 128), g)
    return q, k, v


@pytest.mark.parametrize("G", [1, 2, 4, 5, 8])
def test_dense_causal_matches_oracle(cuda_device, G):
    hkv = 2
    qlens = [1, 17, 64, 65, 200, 333]
    q, k, v = _dense_case(100 + G, qlens, G * hkv, hkv)
    cu = _cu(qlens)
    d = cuda_device
    out = _prefill(q.to(d), k.to(d), v.to(d), cu.to(d), cu.to(d), max(qlens))
    torch.cuda.synchronize()
    want = ref.varlen_prefill(q, k, v, cu, cu, SCALE)
    torch.testing.assert_close(out.cpu().float(), want, **TOL)


def test_dense_noncausal_matches_oracle(cuda_device):
    qlens = [3, 130, 77]
    q, k, v = _dense_case(110, qlens, 16, 8, qkv_view=False)
    cu = _cu(qlens)
    d = cuda_device
    out = _prefill(q.to(d), k.to(d), v.to(d), cu.to(d), cu.to(d), max(qlens), causal=False)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().float(), ref.varlen_prefill(q, k, v, cu, cu, SCALE, causal=False), **TOL)


def _paged_case(seed, qlens, prefix, hq, hkv, bs, layout="interleaved", nb=None):
    g = gen(seed)
    klens = [a + b for a, b in zip(qlens, prefix)]
    need = sum(math.ceil(k / bs) for k in klens)
    nb = nb or need + 5
    if layout == "interleaved":
        _, kc, vc = interleaved_pool(nb, bs, hkv, 128, g)
    else:
        kc, vc = contiguous_caches(nb, bs, hkv, 128, g)
    bt = random_block_tables(klens, bs, nb, g)
    q = randn_bf16((sum(qlens), hq, 128), g)
    return q, kc, vc, bt, _cu(qlens), _cu(klens)


@pytest.mark.parametrize("bs,layout", [(256, "interleaved"), (64, "contiguous")])
@pytest.mark.parametrize("G", [2, 4, 5])
def test_paged_prefix_matches_oracle(cuda_device, bs, layout, G):
    """Prefix-cached prefill over the pages: block-aligned prefixes (prefix-cache hits),
    unaligned ones (chunked prefill, scheduler.py:124) and empty ones in one batch."""
    qlens = [70, 5, 300, 1, 129]
    prefix = [256, 37, 0, 511, 1024]
    q, kc, vc, bt, cq, ck = _paged_case(200 + bs + G, qlens, prefix, G * 2, 2, bs, layout)
    d = cuda_device
    out = _prefill(q.to(d), kc.to(d), vc.to(d), cq.to(d), ck.to(d), max(qlens), bt=bt.to(d))
    torch.cuda.synchronize()
    want = ref.varlen_prefill(q, kc, vc, cq, ck, SCALE, block_tables=bt)
    torch.testing.assert_close(out.cpu().float(), want, **TOL)


def test_paged_equals_dense_bitwise(cuda_device):
    """The same keys read through scattered pages or as packed rows give identical bits."""
    qlens = [40, 300, 9]
    q, kc, vc, bt, cq, ck = _paged_case(210, qlens, [0, 0, 0], 16, 8, 256)
    d = cuda_device
    kd = torch.cat([ref._gather_tokens(kc, bt[s], qlens[s]) for s in range(3)])
    vd = torch.cat([ref._gather_tokens(vc, bt[s], qlens[s]) for s in range(3)])
    paged = _prefill(q.to(d), kc.to(d), vc.to(d), cq.to(d), ck.to(d), max(qlens), bt=bt.to(d))
    dense = _prefill(q.to(d), kd.to(d), vd.to(d), cq.to(d), ck.to(d), max(qlens))
    torch.cuda.synchronize()
    assert bits_equal(paged.cpu(), dense.cpu())


def test_grid_smaller_than_longest_sequence(cuda_device):
    """max_seqlen_q only sizes the grid: an understated value still computes every row."""
    qlens = [500, 20]
    q, k, v = _dense_case(220, qlens, 16, 8)
    cu = _cu(qlens)
    d = cuda_device
    out = _prefill(q.to(d), k.to(d), v.to(d), cu.to(d), cu.to(d), 64)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().float(), ref.varlen_prefill(q, k, v, cu, cu, SCALE), **TOL)


def test_rows_without_keys_and_empty_sequences(cuda_device):
    """klen < qlen leaves leading rows with no visible key (zeros); zero-length
    sequences in the batch are harmless."""
    g = gen(230)
    q = randn_bf16((12, 4, 128), g)
    k, v = randn_bf16((7, 2, 128), g), randn_bf16((7, 2, 128), g)
    cq, ck = _cu([10, 0, 2]), _cu([5, 0, 2])
    d = cuda_device
    out = _prefill(q.to(d), k.to(d), v.to(d), cq.to(d), ck.to(d), 10)
    torch.cuda.synchronize()
    want = ref.varlen_prefill(q, k, v, cq, ck, SCALE)
    torch.testing.assert_close(out.cpu().float(), want, **TOL)
    assert torch.count_nonzero(out[:5].cpu()) == 0


def test_invalid_block_poisons_only_its_sequence(cuda_device):
    qlens, prefix = [50, 60], [256, 256]
    q, kc, vc, bt, cq, ck = _paged_case(240, qlens, prefix, 16, 8, 256)
    bad = bt.clone()
    bad[0, 0] = kc.shape[0] + 3
    d = cuda_device
    out = _prefill(q.to(d), kc.to(d), vc.to(d), cq.to(d), ck.to(d), 60, bt=bad.to(d)).cpu().float()
    assert torch.isnan(out[:50]).all()
    want = ref.varlen_prefill(q, kc, vc, cq, ck, SCALE, block_tables=bt)
    torch.testing.assert_close(out[50:], want[50:], **TOL)


def _config_d(g, nb=4096, bs=256):
    """32 sequences in 8 groups of 4: each group shares a cached prefix of 0-4096 tokens in
    whole 256-token blocks (identical leading block ids), each sequence 100-1024 new tokens
    in its own blocks."""
    qlens, prefix, tables = [], [], []
    perm = torch.randperm(nb, generator=g).tolist()
    pos = 0
    for grp in range(8):
        p = 256 * int(torch.randint(0, 17, (1,), generator=g))
        shared = perm[pos:pos + p // 256]
        pos += p // 256
        for _ in range(4):
            n = int(torch.randint(100, 1025, (1,), generator=g))
            own = perm[pos:pos + math.ceil((p + n) / bs) - len(shared)]
            pos += len(own)
            qlens.append(n)
            prefix.append(p)
            tables.append(shared + own)
    width = max(len(t) for t in tables)
    bt = torch.tensor([t + [-1] * (width - len(t)) for t in tables], dtype=torch.int32)
    return qlens, prefix, bt


def _device_oracle_prefill(q, k, v, cq, ck, out, bt=None):
    """Every sequence against the fp32 oracle, evaluated on the device in float32."""
    allow = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        cqh, ckh = cq.tolist(), ck.tolist()
        for s in range(len(cqh) - 1):
            r0, r1 = cqh[s], cqh[s + 1]
            if bt is None:
                want = ref.varlen_prefill(q[r0:r1], k[ckh[s]:ckh[s + 1]], v[ckh[s]:ckh[s + 1]],
                                          _cu([r1 - r0]), _cu([ckh[s + 1] - ckh[s]]), SCALE)
            else:
                want = ref.varlen_prefill(q[r0:r1], k, v, _cu([r1 - r0]), _cu([ckh[s + 1] - ckh[s]]), SCALE,
                                          block_tables=bt[s:s + 1])
            torch.testing.assert_close(out[r0:r1].float(), want, **TOL, msg=lambda m: f"sequence {s}: {m}")
    finally:
        torch.backends.cuda.matmul.allow_tf32 = allow


def test_full_size_prefix_shared_every_sequence(cuda_device):
    """The prefix-cached prefill workload at full size (32 sequences, 100-1024 new tokens,
    prefixes of 0-4096 tokens shared by groups of 4, Qwen3-0.6B heads).  Every sequence is
    compared with the fp32 oracle, so a unit ranked or dealt wrongly for some sequences of
    the real batch fails here."""
    g = gen(250)
    bs, hkv, hq, d, nb = 256, 8, 16, cuda_device, 4096
    qlens, prefix, bt = _config_d(g, nb, bs)
    cq, ck = _cu(qlens), _cu([a + b for a, b in zip(qlens, prefix)])
    dg = torch.Generator(device=d).manual_seed(250)
    kc = torch.randn(nb, bs, hkv, 128, generator=dg, device=d, dtype=torch.bfloat16)
    vc = torch.randn(nb, bs, hkv, 128, generator=dg, device=d, dtype=torch.bfloat16)
    q = randn_bf16((sum(qlens), hq, 128), g).to(d)
    bt_d = bt.to(d)
    out = _prefill(q, kc, vc, cq.to(d), ck.to(d), max(qlens), bt=bt_d)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    _device_oracle_prefill(q, kc, vc, cq, ck, out, bt=bt_d)
    del kc, vc
    torch.cuda.empty_cache()


def test_full_size_dense_every_sequence(cuda_device):
    """The same 32 sequences' new tokens without prefixes, dense k / v rows (the no-prefix
    batches of the reference's caller, block_table None): every sequence against the
    fp32 oracle."""
    g = gen(251)
    hkv, hq, d = 8, 16, cuda_device
    qlens, _, _ = _config_d(g)
    cq = _cu(qlens)
    dg = torch.Generator(device=d).manual_seed(251)
    q = torch.randn(sum(qlens), hq, 128, generator=dg, device=d, dtype=torch.bfloat16)
    k = torch.randn(sum(qlens), hkv, 128, generator=dg, device=d, dtype=torch.bfloat16)
    v = torch.randn(sum(qlens), hkv, 128, generator=dg, device=d, dtype=torch.bfloat16)
    out = _prefill(q, k, v, cq.to(d), cq.to(d), max(qlens))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    _device_oracle_prefill(q, k, v, cq, cq, out)


def test_prefill_golden(cuda_device):
    f = load("prefill_small")
    d = cuda_device
    cq = torch.from_numpy(f["cu_seqlens_q"])
    out = _prefill(bf16(f["q"]).to(d), bf16(f["k_cache"]).to(d), bf16(f["v_cache"]).to(d),
                   cq.to(d), torch.from_numpy(f["cu_seqlens_k"]).to(d), int(np.diff(f["cu_seqlens_q"]).max()),
                   scale=float(f["scale"]), bt=torch.from_numpy(f["block_tables"]).to(d))
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().double(), torch.from_numpy(f["out"]), **TOL)


def test_paged_table_longer_than_64_blocks(cuda_device):
    """Contexts of more than 64 blocks: block ids come from a 64-entry window held in
    registers, reloaded as the key tiles move into the next window (64-token pages: klen
    4800 = 75 blocks, 9100 = 143 blocks = three windows), and back to the first window
    for each query tile of the sequence."""
    qlens = [300, 40, 200]
    prefix = [4500, 4200, 8900]
    q, kc, vc, bt, cq, ck = _paged_case(250, qlens, prefix, 4, 2, 64)
    assert bt.shape[1] >= 143
    d = cuda_device
    out = _prefill(q.to(d), kc.to(d), vc.to(d), cq.to(d), ck.to(d), max(qlens), bt=bt.to(d))
    torch.cuda.synchronize()
    want = ref.varlen_prefill(q, kc, vc, cq, ck, SCALE, block_tables=bt)
    torch.testing.assert_close(out.cpu().float(), want, **TOL)


def test_paged_block_size_512(cuda_device):
    qlens = [700, 3, 513]
    prefix = [512, 1000, 0]
    q, kc, vc, bt, cq, ck = _paged_case(251, qlens, prefix, 16, 8, 512)
    d = cuda_device
    out = _prefill(q.to(d), kc.to(d), vc.to(d), cq.to(d), ck.to(d), max(qlens), bt=bt.to(d))
    torch.cuda.synchronize()
    want = ref.varlen_prefill(q, kc, vc, cq, ck, SCALE, block_tables=bt)
    torch.testing.assert_close(out.cpu().float(), want, **TOL)


def test_many_sequences_and_query_tile_pairs(cuda_device):
    """Many short sequences and an odd number of query tiles per sequence: the grid pads
    to whole pairs of tiles on every XCD and the extra work items do nothing."""
    g = gen(252)
    qlens = [int(x) for x in torch.randint(1, 200, (67,), generator=g)]
    prefix = [int(x) * 64 for x in torch.randint(0, 5, (67,), generator=g)]
    q, kc, vc, bt, cq, ck = _paged_case(253, qlens, prefix, 8, 4, 64)
    d = cuda_device
    out = _prefill(q.to(d), kc.to(d), vc.to(d), cq.to(d), ck.to(d), max(qlens), bt=bt.to(d))
    torch.cuda.synchronize()
    want = ref.varlen_prefill(q, kc, vc, cq, ck, SCALE, block_tables=bt)
    torch.testing.assert_close(out.cpu().float(), want, **TOL)


def test_dense_persistent_workgroups_take_many_units(cuda_device):
    """Dense prefill runs persistent workgroups.  320 sequences of 1-400 tokens with an
    understated max_seqlen_q (so a unit spans several tile pairs) give each workgroup
    many units of unequal cost.  Every row equals the paged instance's (one unit per
    workgroup) bit for bit, and the oracle within tolerance."""
    g = gen(256)
    qlens = [int(x) for x in torch.randint(1, 401, (320,), generator=g)]
    q, kc, vc, bt, cq, ck = _paged_case(257, qlens, [0] * len(qlens), 16, 8, 64)
    kd = torch.cat([ref._gather_tokens(kc, bt[s], qlens[s]) for s in range(len(qlens))])
    vd = torch.cat([ref._gather_tokens(vc, bt[s], qlens[s]) for s in range(len(qlens))])
    d = cuda_device
    dense = _prefill(q.to(d), kd.to(d), vd.to(d), cq.to(d), cq.to(d), 100)
    paged = _prefill(q.to(d), kc.to(d), vc.to(d), cq.to(d), ck.to(d), 100, bt=bt.to(d))
    torch.cuda.synchronize()
    assert bits_equal(dense.cpu(), paged.cpu())
    torch.testing.assert_close(dense.cpu().float(), ref.varlen_prefill(q, kd, vd, cq, cq, SCALE), **TOL)


def test_paged_relocated_pages_are_bitwise_identical(cuda_device):
    """Prefix-cached prefill over pages moved to other physical blocks (tables renumbered
    to match) gives identical bits."""
    qlens, prefix = [70, 300, 1, 129], [256, 37, 511, 0]
    q, kc, vc, bt, cq, ck = _paged_case(230, qlens, prefix, 16, 8, 256)
    k2, v2, bt2 = relocate_pages(kc, vc, bt, gen(231))
    d = cuda_device
    a = _prefill(q.to(d), kc.to(d), vc.to(d), cq.to(d), ck.to(d), max(qlens), bt=bt.to(d)).cpu()
    b = _prefill(q.to(d), k2.to(d), v2.to(d), cq.to(d), ck.to(d), max(qlens), bt=bt2.to(d)).cpu()
    assert bits_equal(a, b)


@pytest.mark.parametrize("paged", [True, False])
def test_more_sequences_than_one_launch(cuda_device, paged):
    """4100 sequences run as three launches (2048 + 2048 + 4): the later ones read their
    cu_seqlens and block-table rows through offset pointers and write the same absolute
    rows.  Paged, the random tables make sequences share first blocks, so the plan ranks
    groups of up to dozens of sequences together."""
    g = gen(260 + paged)
    nseq, bs, nb = 4100, 64, 64
    qlens = [int(x) for x in torch.randint(1, 4, (nseq,), generator=g)]
    prefix = [int(x) for x in torch.tensor([0, 5, 64])[torch.randint(0, 3, (nseq,), generator=g)]]
    if not paged:
        prefix = [0] * nseq
    klens = [a + b for a, b in zip(qlens, prefix)]
    q = randn_bf16((sum(qlens), 4, 128), g)
    d = cuda_device
    if paged:
        kc, vc = contiguous_caches(nb, bs, 2, 128, g)
        # pages shared between sequences (as prefix-cache hits share them), -1 past the need
        bt = torch.randint(0, nb, (nseq, 2), generator=g, dtype=torch.int32)
        bt[torch.tensor([math.ceil(k / bs) for k in klens]) == 1, 1] = -1
        out = _prefill(q.to(d), kc.to(d), vc.to(d), _cu(qlens).to(d), _cu(klens).to(d), 3, bt=bt.to(d))
        want = ref.varlen_prefill(q, kc, vc, _cu(qlens), _cu(klens), SCALE, block_tables=bt)
    else:
        k = randn_bf16((sum(klens), 2, 128), g)
        v = randn_bf16((sum(klens), 2, 128), g)
        out = _prefill(q.to(d), k.to(d), v.to(d), _cu(qlens).to(d), _cu(klens).to(d), 3)
        want = ref.varlen_prefill(q, k, v, _cu(qlens), _cu(klens), SCALE)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().float(), want, **TOL)


@pytest.mark.parametrize("paged", [False, True])
def test_rising_scores_rebase_the_running_max(cuda_device, paged):
    """P is formed against the running max of the query tile's first key tile; later
    tiles whose scores rise past it re-base the max.  Sequence 0: scores grow by about
    1.5 (base 2) per 64-key tile over 32 tiles, so the max is re-based every dozen tiles.
    Sequence 1: keys after the first tile score about 133 (base 2) above the first ones,
    so exp2 overflows to inf before the re-base.  Both against the oracle."""
    g = gen(270)
    u = torch.zeros(128)
    u[0] = 1.0
    qlens, klens = [64, 64], [2048, 256]
    q = (4.0 * u + 0.05 * torch.randn(sum(qlens), 16, 128, generator=g)).to(torch.bfloat16)
    rise = (3.0 * (torch.arange(2048) // 64).float()).view(-1, 1, 1) * u
    jump = torch.where(torch.arange(256) < 64, 0.0, 260.0).view(-1, 1, 1) * u
    k = torch.cat([rise, jump]).expand(-1, 8, 128) + 0.05 * torch.randn(sum(klens), 8, 128, generator=g)
    k = k.to(torch.bfloat16)
    v = randn_bf16((sum(klens), 8, 128), g)
    cq, ck = _cu(qlens), _cu(klens)
    d = cuda_device
    want = ref.varlen_prefill(q, k, v, cq, ck, SCALE)
    if paged:
        bs, nb = 64, sum(klens) // 64 + 3
        perm = torch.randperm(nb, generator=g)
        kc = torch.zeros(nb, bs, 8, 128, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        tables, pos = [], 0
        for s, kl in enumerate(klens):
            ids = perm[pos:pos + kl // bs]
            pos += kl // bs
            kc[ids] = k[ck[s]:ck[s + 1]].view(-1, bs, 8, 128)
            vc[ids] = v[ck[s]:ck[s + 1]].view(-1, bs, 8, 128)
            tables.append(ids.tolist())
        width = max(len(t) for t in tables)
        bt = torch.tensor([t + [-1] * (width - len(t)) for t in tables], dtype=torch.int32)
        out = _prefill(q.to(d), kc.to(d), vc.to(d), cq.to(d), ck.to(d), 64, bt=bt.to(d))
    else:
        out = _prefill(q.to(d), k.to(d), v.to(d), cq.to(d), ck.to(d), 64)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    torch.testing.assert_close(out.cpu().float(), want, **TOL)


def test_prefill_graph_replay_with_new_data(cuda_device):
    """Prefill captured in a graph after reserving its workspace: each replay's plan kernel
    rewrites the work list and zeroes the claim counters in the workspace (no memset is
    recorded), so replays with new queries, keys and lengths written into the captured
    buffers equal eager calls bit for bit.  Eager work runs between the replays."""
    from kavor_amd.layers.attention import reserve_prefill_workspace, varlen_prefill

    d = cuda_device
    hq, hkv, bs, nb, nseq = 16, 8, 64, 96, 6
    g = gen(280)
    kc = randn_bf16((nb, bs, hkv, 128), g).to(d)
    vc = randn_bf16((nb, bs, hkv, 128), g).to(d)
    width = 16
    q = torch.zeros(6 * 256, hq, 128, dtype=torch.bfloat16, device=d)
    cq = torch.zeros(nseq + 1, dtype=torch.int32, device=d)
    ck = torch.zeros(nseq + 1, dtype=torch.int32, device=d)
    bt = torch.zeros(nseq, width, dtype=torch.int32, device=d)
    out = torch.zeros_like(q)
    max_q = 256
    reserve_prefill_workspace(nseq, max_q, hq, hkv, d)

    def draw(seed):
        g2 = gen(seed)
        qlens = [int(x) for x in torch.randint(1, max_q + 1, (nseq,), generator=g2)]
        prefix = [64 * int(x) for x in torch.randint(0, 6, (nseq,), generator=g2)]
        klens = [a + b for a, b in zip(qlens, prefix)]
        tables = torch.randint(0, nb, (nseq, width), generator=g2, dtype=torch.int32)
        return qlens, klens, tables, randn_bf16((sum(qlens), hq, 128), g2)

    def load(qlens, klens, tables, qd):
        q.zero_()
        q[:qd.shape[0]] = qd.to(d)
        cq.copy_(_cu(qlens))
        ck.copy_(_cu(klens))
        bt.copy_(tables)

    def call():
        return varlen_prefill(q, kc, vc, max_q, cq, 0, ck, SCALE, causal=True, block_table=bt, out=out)

    load(*draw(281))
    call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for rep in range(3):
        qlens, klens, tables, qd = draw(282 + rep)
        load(qlens, klens, tables, qd)
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = out[:sum(qlens)].clone()
        eager = varlen_prefill(q, kc, vc, max_q, cq, 0, ck, SCALE, causal=True, block_table=bt)[:sum(qlens)]
        torch.cuda.synchronize()
        assert bits_equal(got.cpu(), eager.cpu()), f"replay {rep}"
        want = ref.varlen_prefill(qd, kc.cpu(), vc.cpu(), _cu(qlens), _cu(klens), SCALE, block_tables=tables)
        torch.testing.assert_close(got.cpu().float(), want, **TOL)
