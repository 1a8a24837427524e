"""The prefill's work order (varlen_prefill.hip): a Python mirror of the plan kernel
(prefill_plan_kernel) and of the persistent workgroups' claims, checked on the CPU.

The plan kernel histograms the (sequence, pair index j) pairs by their sequence's
key-tile count ceil(kl / 64), turns the histogram into offsets in decreasing level, and
places each pair at the next offset of its level (LDS atomics: pairs of one level land
in no fixed order).  With block tables, sequences whose first block id is the same (a
prefix-cache hit) all take the largest level among them, so they rank together.  Rank r is kv head r % H of pair r // H.  The workgroups of XCD x claim
c = 0, 1, 2, ... from their own counter; claim c is rank 8 (c // 2) + x, member c % 2 (the
earlier tile of the pair), and a member takes query tiles t = 2j + member, t + 2J, ...
counted from the sequence's last tile.  The properties that keep the kernel correct and
fast:

- claims -> (sequence, kv head, query tile) cover every query tile exactly once, whatever
  order the pairs of one level land in, also when max_seqlen_q understates the longest
  sequence (units then stride over tile pairs) and when a pair has no earlier tile;
- the level by rank never increases, every pair of a sequence has the same level, and
  sequences that start with the same block share it;
- a pair's level bounds the key-tile count the kernel's key loop runs for its later
  tile, and equals it for the last pair of the group's longest sequence, so the longest
  sequences start first.

The GPU tests check the kernel's outputs against the oracle on the same shapes."""

import itertools
import math
import random

import pytest
import torch

KEY_TILE = 64
PLAN_LEVELS = 2048
SCALE = 128 ** -0.5


def tile_cost(ql, kl, i, tok, causal):
    """Key tiles of query tile i, as the kernel's key loop counts them."""
    kv_end = kl if not causal else min(kl, min(ql, (i + 1) * tok) + kl - ql)
    return (kv_end + KEY_TILE - 1) // KEY_TILE if kv_end > 0 else 0


def seq_levels(lens, first_blocks=None):
    """Each sequence's level: its key-tile count, or with first block ids (paged) the
    largest one among the sequences with queries that start with the same block (ids < 0
    and sequences without queries or keys rank alone)."""
    def level(kl):
        return min(max(-(-kl // KEY_TILE), 0), PLAN_LEVELS - 1)

    lv = [level(kl) for _, kl in lens]
    if first_blocks is not None:
        top = {}
        joins = [ql > 0 and kl > 0 and first_blocks[s] >= 0 for s, (ql, kl) in enumerate(lens)]
        for s in range(len(lens)):
            if joins[s]:
                top[first_blocks[s]] = max(top.get(first_blocks[s], 0), lv[s])
        lv = [top[first_blocks[s]] if joins[s] else lv[s] for s in range(len(lens))]
    return lv


def plan(lens, tok, causal, pair_slots, rng, first_blocks=None):
    """The plan kernel: pairs (s, j) in decreasing level, ties shuffled (placement order
    within a level is whatever the LDS atomics give)."""
    lv = seq_levels(lens, first_blocks)
    by_level = {}
    for s, (ql, kl) in enumerate(lens):
        nu = min(pair_slots, ((ql + tok - 1) // tok + 1) // 2)
        for j in range(nu):
            by_level.setdefault(lv[s], []).append((s, j))
    pairs = []
    for lv in sorted(by_level, reverse=True):
        group = by_level[lv]
        rng.shuffle(group)
        pairs += [(s, j, lv) for s, j in group]
    return pairs


def check_order(lens, heads, group, causal, max_seqlen_q, rng, first_blocks=None):
    tok = 128 // group
    pair_slots = (math.ceil(max_seqlen_q / tok) + 1) // 2
    pairs = plan(lens, tok, causal, pair_slots, rng, first_blocks)
    num_units = len(pairs) * heads
    levels = [pairs[r // heads][2] for r in range(num_units)]
    assert all(a >= b for a, b in zip(levels, levels[1:]))
    seq_level = {}
    for s, _, lv in pairs:
        assert seq_level.setdefault(s, lv) == lv
    # the level is the largest key-tile count of the sequences sharing the first block,
    # reached by the last pair of the longest of them
    groups = {}
    for s, (q, k) in enumerate(lens):
        key = first_blocks[s] if first_blocks is not None and q > 0 and k > 0 and first_blocks[s] >= 0 else ("alone", s)
        groups.setdefault(key, []).append(s)
    for members in groups.values():
        with_pairs = [s for s in members if s in seq_level]
        assert len({seq_level[s] for s in with_pairs}) <= 1
        if with_pairs:
            longest = max(min(tile_cost(lens[s][0], lens[s][1], (lens[s][0] + tok - 1) // tok - 1, tok, causal),
                              PLAN_LEVELS - 1) for s in members if lens[s][0] > 0)
            assert seq_level[with_pairs[0]] == longest
    seen = set()
    for xcd in range(8):
        c = 0
        while True:
            r = 8 * (c // 2) + xcd
            if r >= num_units:
                break
            member = c % 2
            s, j, lv = pairs[r // heads]
            kvh = r % heads
            q, k = lens[s]
            ntl = (q + tok - 1) // tok
            assert 0 <= j < pair_slots
            cost = min(tile_cost(q, k, ntl - 1 - 2 * j, tok, causal), PLAN_LEVELS - 1)
            assert cost <= lv, (q, k, j, cost, lv)
            t = 2 * j + member
            while t < ntl:  # a member past the last tile has no query tile (an empty unit)
                key = (s, kvh, ntl - 1 - t)
                assert key not in seen, key
                seen.add(key)
                t += 2 * pair_slots
            c += 1
    want = {(s, h, t) for s, (q, _) in enumerate(lens) for h in range(heads) for t in range((q + tok - 1) // tok)}
    assert seen == want


def test_prefix_cached_workload_shape():
    """32 sequences, 100-1024 new tokens over prefixes of 0-4096 shared by groups of 4
    (a shared prefix: the same first block; without one, each sequence its own)."""
    rng = random.Random(0)
    lens, first = [], []
    for g in range(8):
        p = 256 * rng.randint(0, 16)
        lens += [(n, p + n) for n in (rng.randint(100, 1024) for _ in range(4))]
        first += [g] * 4 if p else [100 + 4 * g + i for i in range(4)]
    for order_seed in range(3):
        check_order(lens, 8, 2, True, max(q for q, _ in lens), random.Random(order_seed))
        check_order(lens, 8, 2, True, max(q for q, _ in lens), random.Random(order_seed), first)
    # the four sequences of a prefix group rank next to each other
    pairs = plan(lens, 64, True, 8, random.Random(0), first)
    lv = seq_levels(lens, first)
    for g in range(8):
        members = [s for s in range(32) if first[s] == g]
        if members:
            assert len({lv[s] for s in members}) == 1


def test_random_shapes_edge_cases():
    rng = random.Random(1)
    for _ in range(80):
        group = rng.choice([1, 2, 4, 5, 8])
        heads = rng.choice([1, 2, 8])
        causal = rng.random() < 0.8
        lens = []
        for _ in range(rng.randint(1, 70)):
            q = rng.choice([0, 1, 5, 25, 63, 64, 65, 127, 128, 129, 300]) if rng.random() < 0.5 else rng.randint(0, 400)
            k = q + rng.choice([0, 0, 1, 17, 64, 256, 1000])
            if rng.random() < 0.05:
                k = max(0, q - rng.randint(1, 20))  # fewer keys than queries
            lens.append((q, k))
        max_q = max(q for q, _ in lens)
        if max_q == 0:
            continue
        if rng.random() < 0.2:
            max_q = max(1, max_q // 3)  # understated max_seqlen_q
        check_order(lens, heads, group, causal, max_q, rng)
        # paged: some sequences start with a shared block (ids < 0 rank alone)
        first = [rng.choice([-1, 0, 1, 2, 3]) if rng.random() < 0.5 else 1000 + s for s in range(len(lens))]
        check_order(lens, heads, group, causal, max_q, rng, first)


def test_levels_past_the_histogram_tie_at_the_top():
    """Key lengths beyond 2047 key tiles all rank at the top level; coverage holds."""
    lens = [(64, 200_000), (128, 140_000), (10, 10), (300, 131_000)]
    check_order(lens, 2, 2, True, 300, random.Random(5))


# Workspace layout the plan kernel writes (varlen_prefill.hip): the unit count at int 256,
# the ranked pairs from int 512, 8 ints each (sequence, pair index, q start, q length,
# k start, k length, 0, 0).
WS_COUNT_INT, WS_UNITS_INT, UNIT_INTS = 256, 512, 8


def _read_plan(ws, num_kv_heads):
    w = ws.view(torch.int32).cpu()
    count = int(w[WS_COUNT_INT])
    assert count % num_kv_heads == 0
    npairs = count // num_kv_heads
    return w[WS_UNITS_INT:WS_UNITS_INT + UNIT_INTS * npairs].view(npairs, UNIT_INTS).tolist()


@pytest.mark.gpu
@pytest.mark.parametrize("paged", [True, False])
def test_device_plan_matches_the_mirror(cuda_device, paged):
    """The plan kernel's work list, read back from the workspace after a real call: every
    (sequence, pair) once with its lengths, and levels (the mirror's, with prefix groups by
    first block id when paged) that never increase with rank.  Sequences 0-3 share a prefix
    (first block 7), 4-5 another (first block 3), the rest start with blocks of their own;
    one has no queries."""
    from kavor_amd.layers.attention import reserve_prefill_workspace, varlen_prefill

    d = cuda_device
    hq, hkv, bs, nb, D = 16, 8, 64, 160, 128
    rng = random.Random(7)
    qlens = [rng.randint(1, 300) for _ in range(12)]
    qlens[9] = 0
    prefix = [640] * 4 + [192] * 2 + [0] * 6
    klens = [q + p for q, p in zip(qlens, prefix)]
    width = max(-(-k // bs) for k in klens)
    shared = {0: [7] + list(range(8, 17)), 4: [3, 4, 5]}
    nxt = 20
    tables, first = [], []
    for s, k in enumerate(klens):
        need = -(-k // bs)
        lead = shared[0] if s < 4 else shared[4] if s < 6 else []
        lead = lead[:prefix[s] // bs]
        own = list(range(nxt, nxt + need - len(lead)))
        nxt += len(own)
        row = (lead + own) + [-1] * (width - need)
        tables.append(row)
        first.append(row[0] if need else -1)
    assert nxt <= nb
    g = torch.Generator().manual_seed(8)
    q = torch.randn(sum(qlens), hq, D, generator=g).to(torch.bfloat16).to(d)
    cq = torch.tensor([0] + list(itertools.accumulate(qlens)), dtype=torch.int32, device=d)
    ck = torch.tensor([0] + list(itertools.accumulate(klens)), dtype=torch.int32, device=d)
    if paged:
        kc = torch.randn(nb, bs, hkv, D, generator=g).to(torch.bfloat16).to(d)
        vc = torch.randn(nb, bs, hkv, D, generator=g).to(torch.bfloat16).to(d)
        bt = torch.tensor(tables, dtype=torch.int32, device=d)
    else:
        kc = torch.randn(sum(klens), hkv, D, generator=g).to(torch.bfloat16).to(d)
        vc = torch.randn(sum(klens), hkv, D, generator=g).to(torch.bfloat16).to(d)
        bt = None
    max_q = max(qlens)
    ws = reserve_prefill_workspace(len(qlens), max_q, hq, hkv, d)
    varlen_prefill(q, kc, vc, max_q, cq, max(klens), ck, SCALE, causal=True, block_table=bt)
    torch.cuda.synchronize()
    rows = _read_plan(ws, hkv)

    tok = 128 // (hq // hkv)
    pair_slots = (math.ceil(max_q / tok) + 1) // 2
    lens = list(zip(qlens, klens))
    want = {(s, j) for s, (ql, _) in enumerate(lens) for j in range(min(pair_slots, ((ql + tok - 1) // tok + 1) // 2))}
    got = [(r[0], r[1]) for r in rows]
    assert len(got) == len(set(got)) and set(got) == want
    cqs, cks = cq.tolist(), ck.tolist()
    for s, j, q0, ql, k0, kl, z0, z1 in rows:
        assert (q0, ql, k0, kl, z0, z1) == (cqs[s], qlens[s], cks[s], klens[s], 0, 0)
    lv = seq_levels(lens, first if paged else None)
    levels = [lv[s] for s, _ in got]
    assert all(a >= b for a, b in zip(levels, levels[1:])), levels
    if paged:  # the prefix groups rank as one: their pairs are contiguous in the list
        for members in ({0, 1, 2, 3}, {4, 5}):
            idx = [i for i, (s, _) in enumerate(got) if s in members]
            between = {got[i][0] for i in range(idx[0], idx[-1] + 1)}
            assert all(lv[s] == lv[min(members)] for s in between)
