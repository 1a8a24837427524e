"""The prefill's work order (varlen_prefill.hip): a Python mirror of the plan kernel
(prefill_plan_kernel) and of the persistent workgroups' claims, checked on the CPU.

The plan kernel histograms the (sequence, pair index j) pairs by their sequence's
key-tile count ceil(kl / 64), turns the histogram into offsets in decreasing level, and
places each pair at the next offset of its level (LDS atomics: pairs of one level land
in no fixed order).  Rank r is kv head r % H of pair r // H.  The workgroups of XCD x claim
c = 0, 1, 2, ... from their own counter; claim c is rank 8 (c // 2) + x, member c % 2 (the
earlier tile of the pair), and a member takes query tiles t = 2j + member, t + 2J, ...
counted from the sequence's last tile.  The properties that keep the kernel correct and
fast:

- claims -> (sequence, kv head, query tile) cover every query tile exactly once, whatever
  order the pairs of one level land in, also when max_seqlen_q understates the longest
  sequence (units then stride over tile pairs) and when a pair has no earlier tile;
- the level by rank never increases, and every pair of a sequence has the same level;
- a pair's level bounds the key-tile count the kernel's key loop runs for its later
  tile, and equals it for the sequence's last pair (the longest tile), so the longest
  sequences start first.

The GPU tests check the kernel's outputs against the oracle on the same shapes."""

import math
import random

KEY_TILE = 64
PLAN_LEVELS = 2048


def tile_cost(ql, kl, i, tok, causal):
    """Key tiles of query tile i, as the kernel's key loop counts them."""
    kv_end = kl if not causal else min(kl, min(ql, (i + 1) * tok) + kl - ql)
    return (kv_end + KEY_TILE - 1) // KEY_TILE if kv_end > 0 else 0


def plan(lens, tok, causal, pair_slots, rng):
    """The plan kernel: pairs (s, j) in decreasing level, ties shuffled (placement order
    within a level is whatever the LDS atomics give)."""
    def level(kl):
        return min(max(-(-kl // KEY_TILE), 0), PLAN_LEVELS - 1)

    by_level = {}
    for s, (ql, kl) in enumerate(lens):
        nu = min(pair_slots, ((ql + tok - 1) // tok + 1) // 2)
        for j in range(nu):
            by_level.setdefault(level(kl), []).append((s, j))
    pairs = []
    for lv in sorted(by_level, reverse=True):
        group = by_level[lv]
        rng.shuffle(group)
        pairs += [(s, j, lv) for s, j in group]
    return pairs


def check_order(lens, heads, group, causal, max_seqlen_q, rng):
    tok = 128 // group
    pair_slots = (math.ceil(max_seqlen_q / tok) + 1) // 2
    pairs = plan(lens, tok, causal, pair_slots, rng)
    num_units = len(pairs) * heads
    levels = [pairs[r // heads][2] for r in range(num_units)]
    assert all(a >= b for a, b in zip(levels, levels[1:]))
    seq_level = {}
    for s, _, lv in pairs:
        assert seq_level.setdefault(s, lv) == lv
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
            assert cost <= lv and (j > 0 or cost == lv), (q, k, j, cost, lv)
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
    """32 sequences, 100-1024 new tokens over prefixes of 0-4096 shared by groups of 4."""
    rng = random.Random(0)
    lens = []
    for _ in range(8):
        p = 256 * rng.randint(0, 16)
        lens += [(n, p + n) for n in (rng.randint(100, 1024) for _ in range(4))]
    for order_seed in range(3):
        check_order(lens, 8, 2, True, max(q for q, _ in lens), random.Random(order_seed))


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


def test_levels_past_the_histogram_tie_at_the_top():
    """Key lengths beyond 2047 key tiles all rank at the top level; coverage holds."""
    lens = [(64, 200_000), (128, 140_000), (10, 10), (300, 131_000)]
    check_order(lens, 2, 2, True, 300, random.Random(5))
