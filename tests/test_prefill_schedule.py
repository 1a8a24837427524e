"""The prefill's work order (varlen_prefill.hip, varlen_prefill_kernel): a Python mirror
of the in-kernel ranking, checked on the CPU.  Every workgroup pair takes the unit of
work of its own rank in decreasing cost, found by a binary search over cost levels on
closed-form unit counts.  The properties that keep the kernel correct and fast:

- rank -> (sequence, kv head, unit) covers every query tile exactly once, also when
  max_seqlen_q understates the longest sequence (units then stride over tile pairs);
- the cost by rank never increases;
- the ranked unit's first tile really costs the level the search found.

The GPU tests check the kernel's outputs against the oracle on the same shapes."""

import math
import random

KEY_TILE = 64


def units_ge(ql, kl, level, tok, causal, pair_slots):
    """Units of a sequence whose first (longer) tile needs at least `level` key tiles."""
    ntl = (ql + tok - 1) // tok
    if ntl == 0:
        return 0
    all_units = min(pair_slots, (ntl + 1) // 2)
    if level <= 0:
        return all_units
    x = KEY_TILE * (level - 1)
    if kl <= x:
        return 0
    if not causal:
        return all_units
    y = x - (kl - ql)
    fi = 0 if y <= 0 else y // tok
    return min(all_units, (ntl - 1 - fi) // 2 + 1)


def tile_cost(ql, kl, i, tok, causal):
    """Key tiles of query tile i, as the kernel's key loop counts them."""
    kv_end = kl if not causal else min(kl, min(ql, (i + 1) * tok) + kl - ql)
    return (kv_end + KEY_TILE - 1) // KEY_TILE if kv_end > 0 else 0


def pick(rank, lens, heads, tok, causal, pair_slots):
    """The kernel's search: (sequence, kv head, unit, level) of `rank`, or None."""
    def count(level):
        return heads * sum(units_ge(q, k, level, tok, causal, pair_slots) for q, k in lens)

    if rank >= count(0):
        return None
    kmax = max(k for _, k in lens)
    lo, hi, c_hi = 0, (kmax + KEY_TILE - 1) // KEY_TILE + 1, 0
    while hi - lo > 1:
        mid = (lo + hi) >> 1
        c = count(mid)
        if c > rank:
            lo = mid
        else:
            hi, c_hi = mid, c
    rr = rank - c_hi
    for base in range(0, len(lens), 64):  # one 64-lane chunk of sequences at a time
        chunk = lens[base:base + 64]
        ghi = [units_ge(q, k, lo + 1, tok, causal, pair_slots) for q, k in chunk]
        e = [(units_ge(q, k, lo, tok, causal, pair_slots) - g) * heads for (q, k), g in zip(chunk, ghi)]
        incl = [sum(e[:j + 1]) for j in range(len(e))]
        if rr < incl[-1]:
            w = next(j for j in range(len(e)) if incl[j] > rr)
            rr -= incl[w] - e[w]
            per_head = e[w] // heads
            return base + w, rr // per_head, ghi[w] + rr % per_head, lo
        rr -= incl[-1]
    raise AssertionError("counts disagree")


def check_order(lens, heads, group, causal, max_seqlen_q):
    tok = 128 // group
    pair_slots = (math.ceil(max_seqlen_q / tok) + 1) // 2
    grid_pairs = pair_slots * heads * len(lens)
    seen, levels = set(), []
    for rank in range(grid_pairs):
        unit = pick(rank, lens, heads, tok, causal, pair_slots)
        if unit is None:
            continue
        s, kvh, j, level = unit
        q, k = lens[s]
        ntl = (q + tok - 1) // tok
        assert 0 <= kvh < heads and 0 <= j < pair_slots
        assert tile_cost(q, k, ntl - 1 - 2 * j, tok, causal) == level
        levels.append(level)
        for member in (0, 1):
            t = 2 * j + member
            while t < ntl:
                key = (s, kvh, ntl - 1 - t)
                assert key not in seen, key
                seen.add(key)
                t += 2 * pair_slots
    want = {(s, h, t) for s, (q, _) in enumerate(lens) for h in range(heads) for t in range((q + tok - 1) // tok)}
    assert seen == want
    assert all(a >= b for a, b in zip(levels, levels[1:]))


def test_prefix_cached_workload_shape():
    """32 sequences, 100-1024 new tokens over prefixes of 0-4096 shared by groups of 4."""
    rng = random.Random(0)
    lens = []
    for _ in range(8):
        p = 256 * rng.randint(0, 16)
        lens += [(n, p + n) for n in (rng.randint(100, 1024) for _ in range(4))]
    check_order(lens, 8, 2, True, max(q for q, _ in lens))


def test_random_shapes_edge_cases():
    rng = random.Random(1)
    for _ in range(60):
        group = rng.choice([1, 2, 4, 8])
        heads = rng.choice([1, 2, 8])
        causal = rng.random() < 0.8
        lens = []
        for _ in range(rng.randint(1, 70)):
            q = rng.choice([0, 1, 5, 63, 64, 65, 127, 128, 129, 300]) if rng.random() < 0.5 else rng.randint(0, 400)
            k = q + rng.choice([0, 0, 1, 17, 64, 256, 1000])
            if rng.random() < 0.05:
                k = max(0, q - rng.randint(1, 20))  # fewer keys than queries
            lens.append((q, k))
        max_q = max(q for q, _ in lens)
        if max_q == 0:
            continue
        if rng.random() < 0.2:
            max_q = max(1, max_q // 3)  # understated max_seqlen_q
        check_order(lens, heads, group, causal, max_q)
