"""The bench's algorithmic units (closed forms in bench.py) against the oracle's
counting loops, on random and edge-case inputs."""

import random

import bench
from oracle import kvpath_oracle as ref


def test_decode_bytes_match_oracle():
    rng = random.Random(0)
    for _ in range(50):
        ctx = [rng.choice([0, 1, 255, 256, 257, rng.randint(1, 40000)]) for _ in range(rng.randint(1, 40))]
        hq, hkv = rng.choice([(16, 8), (32, 8), (8, 1), (64, 8)])
        bs = rng.choice([64, 256, 512])
        assert bench.decode_bytes(ctx, hq, hkv, 128, bs) == ref.decode_bytes(ctx, hq, hkv, 128, bs)


def test_fused_decode_bytes_match_oracle():
    rng = random.Random(3)
    for _ in range(50):
        ctx = [rng.choice([1, 2, 255, 256, 257, rng.randint(1, 40000)]) for _ in range(rng.randint(1, 40))]
        hq, hkv = rng.choice([(16, 8), (32, 8), (8, 1), (64, 8)])
        bs = rng.choice([64, 256, 512])
        assert bench.fused_decode_bytes(ctx, hq, hkv, 128, bs) == ref.fused_decode_bytes(ctx, hq, hkv, 128, bs)


def test_append_bytes_match_oracle():
    rng = random.Random(1)
    for _ in range(50):
        slots = [rng.choice([-1, rng.randint(0, 10 ** 6)]) for _ in range(rng.randint(0, 300))]
        assert bench.append_bytes(slots, 8, 128) == ref.append_bytes(slots, 8, 128)
    # the headline append: 3968 valid slots, 128 padding
    assert bench.append_bytes(list(range(3968)) + [-1] * 128, 8, 128) == 32_522_240


def test_prefill_flops_match_oracle():
    rng = random.Random(2)
    for _ in range(40):
        qlens = [rng.randint(1, 700) for _ in range(rng.randint(1, 8))]
        # keys >= queries (prefix-cached) and a few with fewer keys than queries
        klens = [q + rng.choice([0, 0, rng.randint(1, 3000), -rng.randint(0, q - 1)]) for q in qlens]
        cq, ck = [0], [0]
        for q, k in zip(qlens, klens):
            cq.append(cq[-1] + q)
            ck.append(ck[-1] + k)
        assert bench.prefill_flops(cq, ck, 16, 128) == ref.prefill_flops(cq, ck, 16, 128)


def test_prefill_bytes_match_oracle():
    rng = random.Random(4)
    for _ in range(30):
        bs = rng.choice([64, 256])
        nseq = rng.randint(1, 8)
        qlens = [rng.randint(1, 500) for _ in range(nseq)]
        prefix = [bs * rng.randint(0, 4) for _ in range(nseq)]
        klens = [q + p for q, p in zip(qlens, prefix)]
        pool = list(range(200))
        rng.shuffle(pool)
        shared = pool[:4]  # every sequence's prefix pages start with the same block ids
        pos = 4
        tables = []
        for p, k in zip(prefix, klens):
            own = -(-k // bs) - p // bs
            tables.append(shared[:p // bs] + pool[pos:pos + own])
            pos += own
        cq, ck = [0], [0]
        for q, k in zip(qlens, klens):
            cq.append(cq[-1] + q)
            ck.append(ck[-1] + k)
        assert (bench.prefill_bytes(cq, ck, 16, 8, 128, tables, bs)
                == ref.prefill_bytes(cq, ck, 16, 8, 128, tables, bs))
        assert bench.prefill_bytes(cq, cq, 16, 8, 128) == ref.prefill_bytes(cq, cq, 16, 8, 128)
    # the prefix-cached and dense 32-sequence workloads
    ql, kl, tables = bench.prefill_workload()
    cq, ck = [0], [0]
    for q, k in zip(ql, kl):
        cq.append(cq[-1] + q)
        ck.append(ck[-1] + k)
    assert bench.prefill_bytes(cq, ck, 16, 8, 128, tables, 256) == ref.prefill_bytes(cq, ck, 16, 8, 128, tables, 256)
