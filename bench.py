"""Benchmark of the paged KV-cache path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extras] [--no-cpu-baseline]
                    [--no-e2e | --e2e-only] [--e2e-seqs N]

A step is one paged-decode pass over the Qwen3-0.6B decode workload (256 sequences,
16 query / 8 kv heads, head_dim 128, bf16, context lengths uniform over 100-2048,
256-token blocks drawn from a shuffled 4096-block pool), with every input resident in
HBM.  `value` is algorithmic HBM bytes per step / time per step (GB/s), timed with HIP
events on the launch stream over exactly K steps after W warm-up steps (defaults 300
and 100), timed before the extra workloads.

The same run also reports, as extra fields (not the headline): the KV append (4096
tokens x 8 heads x 128 into a [512, 256, 8, 128] cache, 128 padding slots), the
Qwen3-8B decode workload (128 sequences, 32/8 heads, contexts 1024-32768, 20000-block
pool) and the prefix-cached varlen prefill (32 sequences, 100-1024 new tokens, prefixes
of 0-4096 tokens shared by groups of 4).  `cpu_baseline` times the PyTorch-eager CPU
restatement (gather + SDPA in bf16) on a bounded sample of the headline workload.
`e2e_qwen3_0.6b` runs the engine end to end: 256 requests on the Qwen3-0.6B
architecture with random bf16 weights, greedy, prompt and output lengths uniform over
100-1024, reporting output tok/s (sum of max_tokens / wall time, prefill included) and
decode tok/s (decode tokens / decode step time).
"""

from __future__ import annotations

import argparse
import itertools
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "paged-decode HBM GB/s (% of 8 TB/s) + KV-append GB/s; Qwen3-0.6B e2e tok/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
BS, D = 256, 128
SCALE = D ** -0.5


# ----------------------------------------------------------------------------- units

def decode_bytes(context_lens, num_q_heads: int, num_kv_heads: int, head_dim: int, block_size: int) -> int:
    """Algorithmic HBM bytes of one paged-decode call: each cached K and V element once
    (bf16), q read and o written once, plus context_lens and the block-table entries used."""
    ctx = [int(c) for c in context_lens]
    kv_row = num_kv_heads * head_dim * 2
    blocks = sum(-(-c // block_size) for c in ctx)
    return 2 * kv_row * sum(ctx) + 2 * len(ctx) * num_q_heads * head_dim * 2 + 4 * (len(ctx) + blocks)


def fused_decode_bytes(context_lens, num_q_heads: int, num_kv_heads: int, head_dim: int,
                       block_size: int) -> int:
    """Algorithmic HBM bytes of one one-launch decode step: the paged decode's bytes with
    the qkv row read in place of q, the new token's K and V written instead of read, one
    fp32 cos/sin row (4 x head_dim B) and the int32 slot per sequence."""
    B = len(context_lens)
    qkv_extra = B * 2 * num_kv_heads * head_dim * 2  # the qkv row is q plus k and v
    return (decode_bytes(context_lens, num_q_heads, num_kv_heads, head_dim, block_size) + qkv_extra
            + B * (4 * head_dim + 4))


def append_bytes(slot_mapping, num_kv_heads: int, head_dim: int) -> int:
    """Algorithmic HBM bytes of one KV append: K and V of each valid (non-negative) slot
    read once and written once (bf16), plus the int32 slot_mapping."""
    slots = [int(x) for x in slot_mapping]
    valid = sum(1 for x in slots if x >= 0)
    return 4 * valid * num_kv_heads * head_dim * 2 + 4 * len(slots)


def prefill_flops(cu_seqlens_q, cu_seqlens_k, num_q_heads: int, head_dim: int) -> int:
    """Algorithmic flops of bottom-right causal varlen prefill: 4 * Hq * D per unmasked
    (query, key) pair.  A sequence with n queries and k >= n keys has n*k - n(n-1)/2
    such pairs (query i sees k - n + 1 + i keys); with k < n only the last k queries see
    any key, k(k+1)/2 pairs."""
    pairs = 0
    for s in range(len(cu_seqlens_q) - 1):
        n = int(cu_seqlens_q[s + 1]) - int(cu_seqlens_q[s])
        k = int(cu_seqlens_k[s + 1]) - int(cu_seqlens_k[s])
        pairs += n * k - n * (n - 1) // 2 if k >= n else k * (k + 1) // 2
    return 4 * num_q_heads * head_dim * pairs


def prefill_bytes(cu_seqlens_q, cu_seqlens_k, num_q_heads: int, num_kv_heads: int, head_dim: int,
                  block_tables=None, block_size: int = 0) -> int:
    """Algorithmic HBM bytes of one varlen prefill call: q read and o written once
    (Tq * Hq * D * 2 each), every distinct key's K and V row read once (Hkv * D * 2 each;
    with block tables a (block, slot) shared by several sequences counts once, as the
    prefix pages of a group), plus 4 bytes per cu_seqlens entry and block-table entry."""
    cq = [int(x) for x in cu_seqlens_q]
    ck = [int(x) for x in cu_seqlens_k]
    tq = cq[-1] - cq[0]
    if block_tables is None:
        keys = ck[-1] - ck[0]
        entries = 0
    else:
        seen = set()
        entries = 0
        for s in range(len(cq) - 1):
            klen = ck[s + 1] - ck[s]
            nblk = -(-klen // block_size)
            entries += nblk
            for b in range(nblk):
                blk = int(block_tables[s][b])
                seen.update((blk, i) for i in range(min(block_size, klen - b * block_size)))
        keys = len(seen)
    return (2 * tq * num_q_heads * head_dim * 2 + 2 * keys * num_kv_heads * head_dim * 2
            + 4 * (len(cq) + len(ck)) + 4 * entries)


# ----------------------------------------------------------------------------- inputs

def decode_inputs(dev, B, hq, hkv, lo, hi, pool_blocks, seed=0):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
    need = [math.ceil(int(c) / BS) for c in ctx]
    width = max(need)
    perm = torch.randperm(pool_blocks, generator=g)
    bt = torch.full((B, width), -1, dtype=torch.int32)
    pos = 0
    for i, n in enumerate(need):
        bt[i, :n] = perm[pos:pos + n].to(torch.int32)
        pos += n
    dg = torch.Generator(device=dev).manual_seed(seed)
    kc = torch.randn(pool_blocks, BS, hkv, D, generator=dg, device=dev, dtype=torch.bfloat16)
    vc = torch.randn(pool_blocks, BS, hkv, D, generator=dg, device=dev, dtype=torch.bfloat16)
    q = torch.randn(B, hq, D, generator=dg, device=dev, dtype=torch.bfloat16)
    return dict(q=q, kc=kc, vc=vc, ctx=ctx.to(dev), bt=bt.to(dev), ctx_host=ctx, bt_host=bt,
                hq=hq, hkv=hkv)


def time_launches(fn, steps: int, warmup: int):
    """Average ms per call over `steps` calls, HIP events on the current (launch) stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_median(fn, steps: int, warmup: int, groups: int = 5):
    """Median over `groups` groups of HIP-event-timed launches (steps in all), in ms per
    call: one slow group (a clock dip on a long kernel) does not move the figure."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    per = max(1, steps // groups)
    times = []
    for _ in range(groups):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(per):
            fn()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / per)
    return statistics.median(times)


def warm_for(fn, seconds: float) -> None:
    """Runs fn until `seconds` of wall time have passed (synchronising every 10 calls):
    the clocks of a part that was idle take a few hundred milliseconds of full load to
    settle, whatever the launch count."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def time_graph(fn, steps: int, warmup: int, per_graph: int = 20):
    """Average ms per call with `per_graph` calls captured in one graph and the graph
    replayed, for kernels shorter than the host's launch interval (eager launches of a
    few-microsecond kernel measure the Python and launch overhead instead)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    reps = max(1, steps // per_graph)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (reps * per_graph)


# ----------------------------------------------------------------------------- workloads

def bench_decode(dev, steps, warmup, shape):
    from kavor_amd.layers.attention import paged_decode, reserve_decode_workspace
    if shape == "qwen3_0.6b":
        inp = decode_inputs(dev, 256, 16, 8, 100, 2048, 4096)
    else:
        inp = decode_inputs(dev, 128, 32, 8, 1024, 32768, 20000)
    B = inp["q"].shape[0]
    out = torch.empty_like(inp["q"])
    reserve_decode_workspace(B, inp["hq"], D, inp["bt"].shape[1], BS, dev)

    def step():
        paged_decode(inp["q"], inp["kc"], inp["vc"], inp["ctx"], inp["bt"], SCALE, out=out)

    # settle the clocks on wall time before the timed launches (a few warm-up calls of a
    # 0.17 ms kernel leave the part below its sustained clock)
    warm_for(step, 0.5)
    ms = time_launches(step, steps, warmup)
    nbytes = decode_bytes(inp["ctx_host"].tolist(), inp["hq"], inp["hkv"], D, BS)
    return inp, dict(ms=ms, bytes=nbytes, gbs=nbytes / ms / 1e6)


def bench_decode_step(dev, steps, warmup):
    """One Qwen3-0.6B attention layer's decode work at the headline shape (256 sequences,
    16q/8kv heads, contexts U[100, 2048]): the q/k norm + RoPE + append kernel followed by
    paged decode, against the one-launch decode step over the same qkv rows, pools and
    slots.  Graph-replayed, 10 calls per graph."""
    from kavor_amd.engine.qwen3 import rope_cache
    from kavor_amd.layers.attention import paged_decode, paged_decode_fused
    from kavor_amd.layers.fused import qk_norm_rope_append

    inp = decode_inputs(dev, 256, 16, 8, 100, 2048, 4096)
    hq, hkv, B = inp["hq"], inp["hkv"], inp["q"].shape[0]
    ctx, bt = inp["ctx_host"].tolist(), inp["bt_host"]
    slots = torch.tensor([int(bt[b, (c - 1) // BS]) * BS + (c - 1) % BS for b, c in enumerate(ctx)],
                         dtype=torch.int32).to(dev)
    pos = inp["ctx"] - 1
    dg = torch.Generator(device=dev).manual_seed(1)
    qkv = torch.randn(B, (hq + 2 * hkv) * D, generator=dg, device=dev).to(torch.bfloat16)
    qw = (torch.rand(D, generator=dg, device=dev) + 0.5).to(torch.bfloat16)
    kw = (torch.rand(D, generator=dg, device=dev) + 0.5).to(torch.bfloat16)
    table = rope_cache(D, 40960, 1e6, dev)
    q = torch.empty(B, hq, D, dtype=torch.bfloat16, device=dev)
    out = torch.empty_like(q)

    def separate():
        qk_norm_rope_append(qkv, pos, table, qw, kw, 1e-6, hq, hkv, inp["kc"], inp["vc"], slots, q_out=q)
        paged_decode(q, inp["kc"], inp["vc"], inp["ctx"], inp["bt"], SCALE, out=out)

    def fused():
        paged_decode_fused(qkv, table, qw, kw, 1e-6, hq, hkv, inp["kc"], inp["vc"], slots, inp["ctx"],
                           inp["bt"], SCALE, out=out)

    res = {}
    for name, fn in (("separate", separate), ("fused", fused)):
        warm_for(fn, 0.5)
        res[name] = time_graph(fn, steps, warmup, per_graph=10) * 1e3
    nbytes = fused_decode_bytes(ctx, hq, hkv, D, BS)
    del inp
    return dict(separate_us=round(res["separate"], 2), fused_us=round(res["fused"], 2), bytes=nbytes,
                gbs=round(nbytes / res["fused"] / 1e3, 1), frac=round(nbytes / res["fused"] / 1e3 / HBM_PEAK_GBS, 4),
                workload="one Qwen3-0.6B layer's decode: B=256, 16q/8kv, ctx U[100,2048], qkv rows -> "
                         "q/k norm + RoPE + append + paged decode, graph-replayed")


def bench_append(dev, steps, warmup):
    from kavor_amd.layers.attention import store_kvcache

    n, hkv, nb = 4096, 8, 512
    g = torch.Generator().manual_seed(0)
    dg = torch.Generator(device=dev).manual_seed(0)
    kc = torch.randn(nb, BS, hkv, D, generator=dg, device=dev, dtype=torch.bfloat16)
    vc = torch.randn(nb, BS, hkv, D, generator=dg, device=dev, dtype=torch.bfloat16)
    # 24 input sets (384 MiB) rotate so that reads come from HBM, not the 256 MiB MALL
    sets = []
    for _ in range(24):
        slots = torch.cat([torch.randperm(nb * BS, generator=g)[:n - 128].to(torch.int32),
                           torch.full((128,), -1, dtype=torch.int32)])
        sets.append((torch.randn(n, hkv, D, generator=dg, device=dev, dtype=torch.bfloat16),
                     torch.randn(n, hkv, D, generator=dg, device=dev, dtype=torch.bfloat16),
                     slots.to(dev)))
    # One graph replays an append per input set: the timed region then holds GPU work
    # only (an 8-10 us kernel is shorter than a Python-level launch).
    for k, v, s in sets:  # warm-up outside capture
        store_kvcache(k, v, kc, vc, s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for k, v, s in sets:
            store_kvcache(k, v, kc, vc, s)
    # at least 10 replays (240 appends) are timed, after the clocks have settled
    replays = max(10, steps // len(sets))
    warm_for(graph.replay, 0.3)
    ms = time_launches(graph.replay, replays, max(1, warmup // len(sets))) / len(sets)
    nbytes = append_bytes(sets[0][2].cpu().tolist(), hkv, D)
    # The engine's layout: one 1 MiB page per block holding K then V (block stride
    # 2 * 256 * 8 * 128 elements), as the page pool binds it.
    page = 2 * BS * hkv * D
    pool = torch.randn(nb, page, generator=dg, device=dev, dtype=torch.bfloat16)
    kp = pool.as_strided((nb, BS, hkv, D), (page, hkv * D, D, 1), 0)
    vp = pool.as_strided((nb, BS, hkv, D), (page, hkv * D, D, 1), BS * hkv * D)
    for k, v, s in sets:
        store_kvcache(k, v, kp, vp, s)
    torch.cuda.synchronize()
    pgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(pgraph):
        for k, v, s in sets:
            store_kvcache(k, v, kp, vp, s)
    warm_for(pgraph.replay, 0.3)
    paged_ms = time_launches(pgraph.replay, replays, max(1, warmup // len(sets))) / len(sets)
    del pgraph, pool, kp, vp
    # The same bytes moved by a plain device copy (torch's copy kernel), timed the same
    # way: the practical ceiling for a transfer this small on this part.
    valid = n - 128
    srcs = [torch.randn(2, valid, hkv * D, generator=dg, device=dev, dtype=torch.bfloat16)
            for _ in range(len(sets))]
    dsts = [torch.empty_like(x) for x in srcs]
    for x, y in zip(srcs, dsts):
        y.copy_(x)
    torch.cuda.synchronize()
    cgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(cgraph):
        for x, y in zip(srcs, dsts):
            y.copy_(x)
    warm_for(cgraph.replay, 0.3)
    copy_ms = time_launches(cgraph.replay, replays, max(1, warmup // len(sets))) / len(srcs)
    return dict(ms=ms, bytes=nbytes, gbs=nbytes / ms / 1e6, copy_ms=copy_ms, paged_ms=paged_ms)


LAYER_TOKENS = 16384  # one full prefill step of the engine (max_num_batched_tokens)


def layer_inputs(dev, T=LAYER_TOKENS):
    """Qwen3-0.6B layer tensors for T tokens: fused qkv rows, an interleaved page pool
    with one 256-token block per 256 tokens (in shuffled order), residual stream rows,
    gate|up rows, and a [256, 151936] logits block."""
    from kavor_amd.engine.qwen3 import rope_cache

    hq, hkv, H, I = 16, 8, 1024, 3072
    dg = torch.Generator(device=dev).manual_seed(0)
    g = torch.Generator().manual_seed(0)
    nb = T // BS
    page = 2 * BS * hkv * D * 2
    pool = torch.zeros(nb, page, dtype=torch.uint8, device=dev)
    flat = pool.view(torch.bfloat16)
    shape, strides = (nb, BS, hkv, D), (page // 2, hkv * D, D, 1)
    kc = flat.as_strided(shape, strides, 0)
    vc = flat.as_strided(shape, strides, BS * hkv * D)
    blocks = torch.randperm(nb, generator=g)
    slots = (blocks.repeat_interleave(BS) * BS + torch.arange(T) % BS).to(torch.int32)
    return dict(
        qkv=torch.randn(T, (hq + 2 * hkv) * D, generator=dg, device=dev, dtype=torch.bfloat16),
        pos=(torch.arange(T) % 4096).to(torch.int32).to(dev),
        table=rope_cache(D, 40960, 1e6, dev), qw=torch.ones(D, device=dev, dtype=torch.bfloat16),
        kc=kc, vc=vc, slots=slots.to(dev),
        x=torch.randn(T, H, generator=dg, device=dev, dtype=torch.bfloat16),
        res=torch.randn(T, H, generator=dg, device=dev, dtype=torch.bfloat16),
        w=torch.ones(H, device=dev, dtype=torch.bfloat16),
        gu=torch.randn(T, 2 * I, generator=dg, device=dev, dtype=torch.bfloat16),
        logits=torch.randn(256, 151936, generator=dg, device=dev, dtype=torch.bfloat16),
        hq=hq, hkv=hkv, H=H, I=I, T=T)


def layer_algo_bytes(inp) -> dict:
    """Algorithmic HBM bytes per launch of each fused layer kernel."""
    T, hq, hkv, H, I = inp["T"], inp["hq"], inp["hkv"], inp["H"], inp["I"]
    return {
        # read the qkv row, write q, write k and v into the pages, read position and slot
        "qk_norm_rope_append": T * ((hq + 2 * hkv) * D * 2 + hq * D * 2 + 2 * hkv * D * 2 + 8),
        # read x and the residual, write the residual and the output
        "add_rmsnorm": T * H * 2 * 4,
        # read gate|up, write the product
        "silu_mul": T * I * 2 * 3,
        # read the logits rows, write one int64 per row
        "argmax": 256 * 151936 * 2 + 256 * 8,
        # a small decode batch: rows split over several workgroups
        "argmax_16rows": 16 * 151936 * 2 + 16 * 8,
        # Gumbel-max sampling at T = 1 (bound by the Philox noise arithmetic, not HBM):
        # logits and temperatures read, one int64 per row written
        "sample_t1": 256 * 151936 * 2 + 256 * 4 + 256 * 8,
    }


def layer_launchers(inp):
    from kavor_amd.layers import fused

    q_out = torch.empty(inp["T"], inp["hq"], D, device=inp["qkv"].device, dtype=torch.bfloat16)
    out = torch.empty_like(inp["x"])
    s_out = torch.empty(inp["T"], inp["I"], device=inp["x"].device, dtype=torch.bfloat16)
    tok = torch.empty(256, dtype=torch.int64, device=inp["x"].device)
    temps = torch.ones(256, dtype=torch.float32, device=inp["x"].device)
    seed = torch.zeros(1, dtype=torch.int32, device=inp["x"].device)
    return {
        "qk_norm_rope_append": lambda: fused.qk_norm_rope_append(
            inp["qkv"], inp["pos"], inp["table"], inp["qw"], inp["qw"], 1e-6, inp["hq"], inp["hkv"],
            inp["kc"], inp["vc"], inp["slots"], q_out=q_out),
        "add_rmsnorm": lambda: fused.add_rms_norm(inp["x"], inp["res"], inp["w"], 1e-6, out=out),
        "silu_mul": lambda: fused.silu_and_mul(inp["gu"], out=s_out),
        "argmax": lambda: fused.greedy_argmax(inp["logits"], out=tok),
        "argmax_16rows": lambda: fused.greedy_argmax(inp["logits"][:16], out=tok[:16]),
        "sample_t1": lambda: fused.sample(inp["logits"], temps, seed, out=tok),
    }


def bench_layers(dev, steps, warmup):
    """The fused kernels around the path at one full engine prefill step (16384 tokens of
    Qwen3-0.6B) and the greedy argmax over a 256 x 151936 logits block."""
    inp = layer_inputs(dev)
    algo = layer_algo_bytes(inp)
    res = {}
    for name, fn in layer_launchers(inp).items():
        warm_for(fn, 0.3)  # settled clocks before each kernel's timed launches
        # the 16-row argmax (about 6 us) is timed as graph replays, as the engine runs it
        ms = (time_graph if name == "argmax_16rows" else time_launches)(fn, steps, warmup)
        res[name] = dict(us=round(ms * 1e3, 2), gbs=round(algo[name] / ms / 1e6, 1),
                         frac=round(algo[name] / ms / 1e6 / HBM_PEAK_GBS, 4), bytes=algo[name])
    res["workload"] = (f"{inp['T']} tokens, Qwen3-0.6B layer (16q/8kv heads, hidden 1024, intermediate "
                       "3072); argmax over [256, 151936] and [16, 151936] bf16 logits; sample_t1: "
                       "Gumbel-max sampling of the [256, 151936] block at T = 1 (Philox noise per value; "
                       "its seed advance included)")
    return res


def prefill_workload(seed: int = 0):
    """Config D's draws: 8 groups of 4 sequences, each group sharing a 256-aligned prefix
    of 0-4096 tokens (identical leading block ids), each sequence 100-1024 new tokens in
    its own blocks; returns (qlens, klens, tables) over a shuffled pool of 4096 blocks."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(4096, generator=g).tolist()
    qlens, klens, tables, pos = [], [], [], 0
    for _ in range(8):
        p = 256 * int(torch.randint(0, 17, (1,), generator=g))
        shared = perm[pos:pos + p // BS]
        pos += p // BS
        for _ in range(4):
            n = int(torch.randint(100, 1025, (1,), generator=g))
            own = perm[pos:pos + math.ceil((p + n) / BS) - len(shared)]
            pos += len(own)
            qlens.append(n)
            klens.append(p + n)
            tables.append(shared + own)
    return qlens, klens, tables


def bench_prefill(dev, steps, warmup, dense: bool = False):
    """Config D (paged, prefix-cached); with dense=True the same new tokens without their
    prefixes, k / v given as packed [tokens, 8, 128] rows (the no-prefix batches of the
    reference's caller, flash_attention_kvcache.py:76-79 with block_table None)."""
    from kavor_amd.layers.attention import varlen_prefill
    hq, hkv, nb = 16, 8, 4096
    qlens, klens, tables = prefill_workload()
    if dense:
        klens = list(qlens)
    width = max(len(t) for t in tables)
    bt = torch.tensor([t + [-1] * (width - len(t)) for t in tables], dtype=torch.int32, device=dev)
    cq = torch.tensor([0] + list(torch.tensor(qlens).cumsum(0)), dtype=torch.int32, device=dev)
    ck = torch.tensor([0] + list(torch.tensor(klens).cumsum(0)), dtype=torch.int32, device=dev)
    dg = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(sum(qlens), hq, D, generator=dg, device=dev, dtype=torch.bfloat16)
    if dense:
        kc = torch.randn(sum(qlens), hkv, D, generator=dg, device=dev, dtype=torch.bfloat16)
        vc = torch.randn(sum(qlens), hkv, D, generator=dg, device=dev, dtype=torch.bfloat16)
        bt = None
    else:
        kc = torch.randn(nb, BS, hkv, D, generator=dg, device=dev, dtype=torch.bfloat16)
        vc = torch.randn(nb, BS, hkv, D, generator=dg, device=dev, dtype=torch.bfloat16)
    out = torch.empty_like(q)

    def step():
        varlen_prefill(q, kc, vc, max(qlens), cq, max(klens), ck, SCALE, causal=True, block_table=bt, out=out)

    warm_for(step, 0.5)
    ms = time_median(step, steps, warmup)
    flops = prefill_flops(cq.cpu().tolist(), ck.cpu().tolist(), hq, D)
    nbytes = prefill_bytes(cq.cpu().tolist(), ck.cpu().tolist(), hq, hkv, D,
                           None if dense else tables, BS)
    return dict(ms=ms, flops=flops, tflops=flops / ms / 1e9, bytes=nbytes, gbs=nbytes / ms / 1e6)


def _median_runs(fn, budget_s: float, min_runs: int = 3, max_runs: int = 50) -> tuple[float, int]:
    fn()  # warm-up
    times, t_end = [], time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def host_cpu() -> dict:
    """The host the CPU baselines run on: threads torch uses (`cores`), the logical CPUs
    the OS reports and the CPU model name."""
    model = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(cores=torch.get_num_threads(), cpu_count=os.cpu_count(), cpu_model=model)


def cpu_baseline_append(budget_s: float = 8.0):
    """The oracle's PyTorch-eager index-put on the host cores, whole config A."""
    from oracle.kvpath_oracle import torch_append

    n, hkv, nb = 4096, 8, 512
    g = torch.Generator().manual_seed(0)
    kc = torch.randn(nb, BS, hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, BS, hkv, D, generator=g).to(torch.bfloat16)
    key = torch.randn(n, hkv, D, generator=g).to(torch.bfloat16)
    value = torch.randn(n, hkv, D, generator=g).to(torch.bfloat16)
    slots = torch.cat([torch.randperm(nb * BS, generator=g)[:n - 128].to(torch.int32),
                       torch.full((128,), -1, dtype=torch.int32)])
    sec, runs = _median_runs(lambda: torch_append(key, value, kc, vc, slots), budget_s)
    nbytes = append_bytes(slots.tolist(), hkv, D)
    return dict(value=round(nbytes / sec / 1e9, 3), unit="GB/s", **host_cpu(), kind="port",
                sample=f"whole workload (4096 tokens, 128 padding), torch {torch.__version__} index-put, "
                       f"median of {runs} runs")


def cpu_baseline_prefill(budget_s: float = 15.0, nseq: int = 4):
    """The oracle's per-sequence gather + masked bf16 SDPA on the host cores, over the
    first sequences of the prefix-cached prefill workload."""
    from oracle.kvpath_oracle import sdpa_varlen_prefill

    hq, hkv = 16, 8
    qlens, klens, tables = prefill_workload()  # the same draws as bench_prefill
    g = torch.Generator().manual_seed(1)
    qlens, klens, tables = qlens[:nseq], klens[:nseq], tables[:nseq]
    ids = sorted({b for t in tables for b in t})
    remap = {b: i for i, b in enumerate(ids)}
    width = max(len(t) for t in tables)
    bt = torch.tensor([[remap[b] for b in t] + [-1] * (width - len(t)) for t in tables], dtype=torch.int32)
    kc = torch.randn(len(ids), BS, hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(len(ids), BS, hkv, D, generator=g).to(torch.bfloat16)
    q = torch.randn(sum(qlens), hq, D, generator=g).to(torch.bfloat16)
    cq = torch.tensor([0] + list(torch.tensor(qlens).cumsum(0)), dtype=torch.int32)
    ck = torch.tensor([0] + list(torch.tensor(klens).cumsum(0)), dtype=torch.int32)
    sec, runs = _median_runs(lambda: sdpa_varlen_prefill(q, kc, vc, cq, ck, SCALE, block_tables=bt), budget_s)
    flops = prefill_flops(cq.tolist(), ck.tolist(), hq, D)
    return dict(value=round(flops / sec / 1e12, 4), unit="TFLOP/s", **host_cpu(), kind="port",
                sample=f"first {nseq} of 32 sequences ({sum(qlens)} query tokens, {sum(klens)} keys), "
                       f"torch {torch.__version__} bf16 SDPA with an explicit bottom-right mask, "
                       f"median of {runs} runs")


def cpu_baseline_decode(inp, budget_s: float = 20.0, nseq: int = 32):
    """The oracle's bf16 gather + SDPA (a PyTorch-eager port of the reference path) on the
    host cores, over the first `nseq` sequences of a decode workload."""
    from oracle.kvpath_oracle import sdpa_paged_decode

    # torch keeps its default thread count (OMP_NUM_THREADS, the host's CPU share)
    ctx = inp["ctx_host"][:nseq]
    bt = inp["bt_host"][:nseq]
    ids = sorted({int(x) for x in bt.flatten() if x >= 0})
    remap = {b: i for i, b in enumerate(ids)}
    sel = torch.tensor(ids, dtype=torch.long, device=inp["kc"].device)
    kc, vc = inp["kc"][sel].cpu(), inp["vc"][sel].cpu()
    bt_c = bt.clone().apply_(lambda x: remap.get(x, -1))
    q = inp["q"][:nseq].cpu()
    sdpa_paged_decode(q, kc, vc, bt_c, ctx, SCALE)  # warm-up
    times, t_end = [], time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        sdpa_paged_decode(q, kc, vc, bt_c, ctx, SCALE)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end and len(times) >= 5:
            break
    sec = statistics.median(times)
    nbytes = decode_bytes(ctx.tolist(), inp["hq"], inp["hkv"], D, BS)
    return dict(value=round(nbytes / sec / 1e9, 4), unit="GB/s", **host_cpu(),
                kind="port",
                sample=f"first {nseq} of {inp['q'].shape[0]} sequences ({int(ctx.sum())} cached tokens), "
                       f"torch {torch.__version__} bf16 SDPA on {platform.processor() or platform.machine()}, "
                       f"median of {len(times)} runs")


def cpu_baseline_e2e(nseq: int = 16, steps: int = 3):
    """A fixed window of the end-to-end workload on the host cores: greedy decode steps
    of the Qwen3-0.6B architecture for the first `nseq` requests, their caches at the
    prompt lengths, computed with the oracle's layer restatements, its PyTorch-eager
    index-put append and its bf16 gather + SDPA attention.  The weights are the engine's
    own (initialised on the GPU with the engine's seed, then copied to the host).
    Returns decode tok/s over the window (comparable to decode_tok_s)."""
    import torch.nn.functional as F

    from kavor_amd.engine.qwen3 import Qwen3ForCausalLM, Qwen3Spec
    from oracle import layers_oracle as L
    from oracle.kvpath_oracle import sdpa_paged_decode, torch_append

    spec = Qwen3Spec()
    model = Qwen3ForCausalLM(spec, "cuda")
    model.init_random(0)
    model = model.to("cpu")
    torch.cuda.empty_cache()
    eps, hq, hkv = spec.rms_norm_eps, spec.num_attention_heads, spec.num_key_value_heads
    prompts, _ = e2e_workload()
    ctx = torch.tensor([len(p) for p in prompts[:nseq]], dtype=torch.int32)
    nblk = [math.ceil((int(c) + steps + 1) / BS) for c in ctx]
    width = max(nblk)
    bt = torch.full((nseq, width), -1, dtype=torch.int32)
    first = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = torch.arange(first, first + n, dtype=torch.int32)
        first += n
    g = torch.Generator().manual_seed(0)
    caches = [tuple((torch.randn(first, BS, hkv, D, generator=g) * 0.5).to(torch.bfloat16) for _ in range(2))
              for _ in range(spec.num_hidden_layers)]
    rows = torch.arange(nseq)

    @torch.inference_mode()
    def decode_step(ids, ctx):
        pos = ctx.long()
        slots = (bt[rows, pos // BS].long() * BS + pos % BS).to(torch.int32)
        h, residual = F.embedding(ids, model.embed_tokens), None
        for layer, (kc, vc) in zip(model.layers, caches):
            if residual is None:
                x, residual = L.rms_norm(h, layer.input_layernorm.weight, eps), h
            else:
                x, residual = L.add_rms_norm(h, residual, layer.input_layernorm.weight, eps)
            a = layer.self_attn
            q, k, v = L.qk_norm_rope(F.linear(x, a.qkv_proj), pos, model.rope_table, a.q_norm.weight,
                                     a.k_norm.weight, eps, hq, hkv)
            torch_append(k, v, kc, vc, slots)
            o = sdpa_paged_decode(q, kc, vc, bt, ctx + 1, D ** -0.5)
            x, residual = L.add_rms_norm(F.linear(o.reshape(nseq, -1), a.o_proj), residual,
                                         layer.post_attention_layernorm.weight, eps)
            h = F.linear(L.silu_and_mul(F.linear(x, layer.mlp.gate_up_proj)), layer.mlp.down_proj)
        x, _ = L.add_rms_norm(h, residual, model.norm.weight, eps)
        return L.greedy(F.linear(x, model.lm_head)), ctx + 1

    ids = torch.tensor([p[-1] for p in prompts[:nseq]], dtype=torch.int64)
    ids, ctx = decode_step(ids, ctx)  # warm-up step
    t0 = time.perf_counter()
    for _ in range(steps):
        ids, ctx = decode_step(ids, ctx)
    sec = time.perf_counter() - t0
    return dict(value=round(nseq * steps / sec, 2), unit="decode tok/s", **host_cpu(),
                kind="port",
                sample=f"{steps} greedy decode steps (after 1 warm-up) of the first {nseq} of 256 requests, "
                       f"engine weights, "
                       f"caches at their prompt lengths ({int(ctx.sum()) - nseq * (steps + 1)} tokens); "
                       f"oracle layers + index-put append + bf16 gather/SDPA attention, torch "
                       f"{torch.__version__}")


def load_traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled
    by the plain-copy calibration), committed as profiles/<name>.json; None if absent."""
    path = ROOT / "profiles" / f"{name}.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get("traffic_bytes")
    except (ValueError, OSError):
        return None


def extra_counts(steps: int, warmup: int) -> dict:
    """Timed and warm-up launches of each extra workload: enough work after warm-up that
    the clocks have settled (a 0.5 ms prefill timed 10 times right after 2 warm-ups reads
    7-15% slow on this part)."""
    return dict(append=(steps, warmup), prefill=(max(20, steps // 3), max(10, warmup // 3)),
                layers=(max(20, steps // 2), max(10, warmup // 3)),
                decode_8b=(max(20, steps // 4), max(5, warmup // 6)))


def run_extras(dev, steps: int, warmup: int, cpu_baseline: bool = False) -> dict:
    n = extra_counts(steps, warmup)
    extras = {}
    a = bench_append(dev, *n["append"])
    extras["kv_append"] = dict(gbs=round(a["gbs"], 1), frac=round(a["gbs"] / HBM_PEAK_GBS, 4),
                               us=round(a["ms"] * 1e3, 3), bytes=a["bytes"],
                               same_bytes_device_copy_us=round(a["copy_ms"] * 1e3, 3),
                               page_interleaved=dict(us=round(a["paged_ms"] * 1e3, 3),
                                                     gbs=round(a["bytes"] / a["paged_ms"] / 1e6, 1)),
                               workload="4096 tok x 8 kv heads x 128 bf16, 3968 valid + 128 pad slots, "
                                        "cache [512,256,8,128] (page_interleaved: the engine's K/V-per-"
                                        "page pool, block stride 2x), 24 rotating input sets, graph-replayed")
    torch.cuda.empty_cache()
    p = bench_prefill(dev, *n["prefill"])
    extras["varlen_prefill"] = dict(tflops=round(p["tflops"], 1), frac=round(p["tflops"] / BF16_PEAK_TFLOPS, 4),
                                    ms=round(p["ms"], 4), flops=p["flops"], bytes=p["bytes"],
                                    intensity_flop_per_byte=round(p["flops"] / p["bytes"], 1),
                                    hbm_gbs=round(p["gbs"], 1), hbm_frac=round(p["gbs"] / HBM_PEAK_GBS, 4),
                                    workload="32 seqs, new 100-1024, prefix 0-4096 shared by groups of 4, 16q/8kv")
    torch.cuda.empty_cache()
    p = bench_prefill(dev, *n["prefill"], dense=True)
    # below the ridge point (2.5 PFLOP/s / 8 TB/s = 312 flop/B) the HBM bound is the roofline
    extras["varlen_prefill_dense"] = dict(tflops=round(p["tflops"], 1), frac=round(p["tflops"] / BF16_PEAK_TFLOPS, 4),
                                          ms=round(p["ms"], 4), flops=p["flops"], bytes=p["bytes"],
                                          intensity_flop_per_byte=round(p["flops"] / p["bytes"], 1),
                                          hbm_gbs=round(p["gbs"], 1), hbm_frac=round(p["gbs"] / HBM_PEAK_GBS, 4),
                                          bound="hbm" if p["flops"] / p["bytes"] < BF16_PEAK_TFLOPS / HBM_PEAK_GBS * 1e3
                                          else "mfma",
                                          workload="config D's 32 sequences of 100-1024 new tokens without "
                                                   "prefixes, dense k/v rows (block_table None), 16q/8kv")
    torch.cuda.empty_cache()
    extras["layer_kernels"] = bench_layers(dev, *n["layers"])
    torch.cuda.empty_cache()
    extras["decode_step_fused"] = bench_decode_step(dev, *n["layers"])
    torch.cuda.empty_cache()
    inp8, c = bench_decode(dev, *n["decode_8b"], "qwen3_8b")
    extras["paged_decode_qwen3_8b"] = dict(gbs=round(c["gbs"], 1), frac=round(c["gbs"] / HBM_PEAK_GBS, 4),
                                           ms=round(c["ms"], 4), bytes=c["bytes"],
                                           workload="B=128, 32q/8kv, ctx U[1024,32768], pool 20000 blocks")
    if cpu_baseline:
        extras["paged_decode_qwen3_8b"]["cpu_baseline"] = cpu_baseline_decode(inp8, budget_s=10.0, nseq=4)
    del inp8
    torch.cuda.empty_cache()
    return extras


def profile_run(dev, steps: int, warmup: int) -> int:
    """The default bench's kernel launches, for rocprofv3: three plain 1 GiB copies first
    (the calibration of the byte counters), then the headline decode and every extra
    workload with the same launch counts as the timed run (no CPU baseline, no engine)."""
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)  # calibration copies
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    bench_decode(dev, steps, warmup, "qwen3_0.6b")
    torch.cuda.empty_cache()
    run_extras(dev, steps, warmup)
    torch.cuda.synchronize()
    print("profile run done", flush=True)
    return 0


PROFILE_CMDS = [
    "cd /tmp && export TMPDIR=/tmp",
    "rocprofv3 --kernel-trace --stats --output-format csv -d $OUT/pmc_trace -o run -- python $R/bench.py --profile",
    "rocprofv3 --pmc FETCH_SIZE --output-format csv -d $OUT/pmc_fetch -o run -- python $R/bench.py --profile",
    "rocprofv3 --pmc WRITE_SIZE --output-format csv -d $OUT/pmc_write -o run -- python $R/bench.py --profile",
    "python $R/bench.py --summarize $OUT/pmc_trace $OUT/pmc_fetch $OUT/pmc_write",
]

PREFILL_PMC_PASSES = [
    "SQ_VALU_MFMA_BUSY_CYCLES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA "
    "SQ_INSTS_VALU_MFMA_MOPS_BF16 SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE GRBM_GUI_ACTIVE",
    "SQ_WAIT_INST_ANY SQ_WAIT_ANY SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_ACTIVE_INST_MISC "
    "SQ_INSTS_LDS SQ_CYCLES SQ_WAIT_INST_LDS GRBM_GUI_ACTIVE",
    "SQ_INSTS_LDS_LOAD_BANDWIDTH SQ_LDS_IDX_ACTIVE TA_TA_BUSY TA_ADDR_STALLED_BY_TC_CYCLES TD_TD_BUSY "
    "TD_TC_STALL GRBM_GUI_ACTIVE",
]
PREFILL_PMC_CMDS = [
    "cd /tmp && export TMPDIR=/tmp",
    "rocprofv3 --pmc " + PREFILL_PMC_PASSES[0] + " --output-format csv -d $OUT/ppmc_a -o run -- "
    "python $R/bench.py --profile-prefill",
    "rocprofv3 --pmc " + PREFILL_PMC_PASSES[1] + " --output-format csv -d $OUT/ppmc_b -o run -- "
    "python $R/bench.py --profile-prefill",
    "rocprofv3 --pmc " + PREFILL_PMC_PASSES[2] + " --output-format csv -d $OUT/ppmc_c -o run -- "
    "python $R/bench.py --profile-prefill",
    "python $R/bench.py --summarize-prefill-pmc $OUT/ppmc_a $OUT/ppmc_b $OUT/ppmc_c",
]


def summarize_prefill_pmc(dir_a: str, dir_b: str, dir_c: str) -> int:
    """profiles/varlen_prefill_prefix_32seq_pmc.md: where the prefill kernel's cycles go,
    from three rocprofv3 --pmc passes over --profile-prefill (medians over the dispatches
    after the first third).  Counters are summed over the device; GRBM_GUI_ACTIVE counts
    once per XCD, so one XCD's busy cycles are its sum divided by the XCD count."""
    import csv
    from collections import defaultdict

    name = "void kvp::varlen_prefill_kernel<2, true, true>"
    vals = defaultdict(lambda: defaultdict(float))
    agent = {}
    for d in (dir_a, dir_b, dir_c):
        for r in csv.DictReader(open(Path(d) / "run_counter_collection.csv")):
            if r["Kernel_Name"].startswith(name):
                vals[(d, int(r["Dispatch_Id"]))][r["Counter_Name"]] += float(r["Counter_Value"])
        for r in csv.DictReader(open(Path(d) / "run_agent_info.csv")):
            if r.get("Name", "").startswith("gfx"):
                agent = r
    cus, simds, xcds = int(agent["Cu_Count"]), int(agent["Simd_Count"]), int(agent["Num_Xcc"])

    def med(counter):
        per = [v[counter] for (d, _), v in sorted(vals.items()) if counter in v]
        per = per[len(per) // 3:]
        return (statistics.median(per), len(per)) if per else (float("nan"), 0)

    gui_a, n = med("GRBM_GUI_ACTIVE")
    xcd_cycles = gui_a / xcds
    mfma_busy = med("SQ_VALU_MFMA_BUSY_CYCLES")[0] / (xcd_cycles * simds)
    waves_per_simd = med("SQ_WAVE_CYCLES")[0] / xcd_cycles / cus
    g = torch.Generator().manual_seed(0)
    perm = torch.randperm(4096, generator=g).tolist()  # the bench_prefill draws
    qlens, klens = [], []
    for _ in range(8):
        p = 256 * int(torch.randint(0, 17, (1,), generator=g))
        for _ in range(4):
            nq = int(torch.randint(100, 1025, (1,), generator=g))
            qlens.append(nq)
            klens.append(p + nq)
    del perm
    cq = [0] + list(torch.tensor(qlens).cumsum(0).tolist())
    ck = [0] + list(torch.tensor(klens).cumsum(0).tolist())
    algo = prefill_flops(cq, ck, 16, D)
    mfma_flops = med("SQ_INSTS_VALU_MFMA_MOPS_BF16")[0] * 512
    lds_conf = med("SQ_LDS_BANK_CONFLICT")[0] / max(1.0, med("SQ_LDS_IDX_ACTIVE")[0])
    wave_cycles = med("SQ_WAVE_CYCLES")[0]
    lines = [
        f"# varlen_prefill_prefix_32seq counters: `{name}(kvp::PrefillParams)`",
        "",
        "Commands (from the repository root on the GPU host, `R=$PWD`, `OUT` a directory for the raw results):",
        "",
        "```",
        *PREFILL_PMC_CMDS,
        "```",
        "",
        f"Device: {agent.get('Name')} with {cus} CUs, {simds} SIMDs, {xcds} XCDs. Medians over the last {n} "
        "of the profiled dispatches. GRBM_GUI_ACTIVE is summed over the XCDs, so one XCD's busy cycles "
        f"= GRBM_GUI_ACTIVE / {xcds}.",
        "",
        "| Quantity | Value | From |",
        "|---|---|---|",
        f"| busy cycles per XCD | {xcd_cycles:,.0f} | GRBM_GUI_ACTIVE / {xcds} |",
        f"| MFMA busy | {100 * mfma_busy:.1f}% of SIMD cycles | SQ_VALU_MFMA_BUSY_CYCLES / (cycles x {simds}) |",
        f"| resident waves per SIMD | {waves_per_simd:.2f} of 2 (VGPR-bound occupancy) | "
        f"SQ_WAVE_CYCLES / cycles / {cus} |",
        f"| MFMA flops executed | {mfma_flops:.4g} = {mfma_flops / algo:.2f} x the algorithmic {algo:.4g} "
        "(the rest: masked halves of diagonal tiles, padded rows of the last query tile) | "
        "SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 |",
        f"| VALU / MFMA / LDS instructions | {med('SQ_INSTS_VALU')[0]:,.0f} / {med('SQ_INSTS_MFMA')[0]:,.0f} / "
        f"{med('SQ_INSTS_LDS')[0]:,.0f} | SQ_INSTS_VALU, SQ_INSTS_MFMA, SQ_INSTS_LDS |",
        f"| LDS bank-conflict cycles | {100 * lds_conf:.1f}% of LDS active cycles | "
        "SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE |",
        f"| waves waiting on a dependency | {100 * med('SQ_WAIT_INST_ANY')[0] / wave_cycles:.1f}% of wave cycles "
        f"(LDS: {100 * med('SQ_WAIT_INST_LDS')[0] / wave_cycles:.1f}%) | SQ_WAIT_INST_ANY, SQ_WAIT_INST_LDS "
        "/ SQ_WAVE_CYCLES |",
        f"| VALU / LDS issue | {100 * med('SQ_ACTIVE_INST_VALU')[0] / wave_cycles:.1f}% / "
        f"{100 * med('SQ_ACTIVE_INST_LDS')[0] / wave_cycles:.1f}% of wave cycles | SQ_ACTIVE_INST_VALU, "
        "SQ_ACTIVE_INST_LDS / SQ_WAVE_CYCLES |",
        f"| LDS reads | {med('SQ_INSTS_LDS_LOAD_BANDWIDTH')[0] * 64 / 1e9:.2f} GB per call = "
        f"{med('SQ_INSTS_LDS_LOAD_BANDWIDTH')[0] * 64 / (xcd_cycles * cus):.1f} B per cycle per CU "
        "(MFMA operands; the tiles' direct-to-LDS writes come on top) | SQ_INSTS_LDS_LOAD_BANDWIDTH x 64 B |",
        f"| texture address / data units busy | {100 * med('TA_TA_BUSY')[0] / (xcd_cycles * cus):.1f}% / "
        f"{100 * med('TD_TD_BUSY')[0] / (xcd_cycles * cus):.1f}% of cycles per CU (TD waiting on the "
        f"L1: {100 * med('TD_TC_STALL')[0] / (xcd_cycles * cus):.1f}%) | TA_TA_BUSY, TD_TD_BUSY, TD_TC_STALL "
        "/ (cycles x CUs) |",
    ]
    out = ROOT / "profiles" / "varlen_prefill_prefix_32seq_pmc.md"
    out.write_text("\n".join(lines) + "\n")
    print(f"wrote {out}", flush=True)
    return 0


# (profile file, kernel-name prefix, which occurrence group, algorithmic bytes or flops, unit)
PROFILE_KERNELS = [
    ("paged_decode_qwen3_0.6b", "void kvp::paged_decode_kernel<2, 32, false>", "decode_0.6b"),
    ("paged_decode_fused_qwen3_0.6b", "void kvp::paged_decode_kernel<2, 32, true>", "decode_fused_0.6b"),
    ("paged_decode_qwen3_8b", "void kvp::paged_decode_kernel<4, 32, false>", "decode_8b"),
    ("kv_append_4096tok", "void kvp::kv_append_kernel<128", "append"),
    ("varlen_prefill_prefix_32seq", "void kvp::varlen_prefill_kernel<2, true, true>", "prefill"),
    ("varlen_prefill_dense_32seq", "void kvp::varlen_prefill_kernel<2, false, true>", "prefill_dense"),
    ("qk_norm_rope_append_16384tok", "void kvp::(anonymous namespace)::qk_norm_rope_append_kernel<4>", "qk_norm_rope_append"),
    ("add_rmsnorm_16384x1024", "void kvp::(anonymous namespace)::rmsnorm_kernel<64, 2>", "add_rmsnorm"),
    ("silu_mul_16384x3072", "kvp::(anonymous namespace)::silu_mul_kernel", "silu_mul"),
    ("argmax_256x151936", "void kvp::(anonymous namespace)::argmax_kernel<1024, 3, false, false>", "argmax"),
    ("sample_256x151936", "void kvp::(anonymous namespace)::argmax_kernel<1024, 3, false, true>", "sample_t1"),
]


def summarize_profiles(trace_dir: str, fetch_dir: str, write_dir: str) -> int:
    """Per-kernel duration and HBM traffic from the three rocprofv3 runs of --profile.

    FETCH_SIZE / WRITE_SIZE (KiB per dispatch) are scaled by what they read for the plain
    1 GiB device copies that start the run (largest __amd_rocclr_copyBuffer dispatches)."""
    import csv
    from collections import defaultdict

    def rows(d, name):
        with open(Path(d) / name) as f:
            return list(csv.DictReader(f))

    trace = rows(trace_dir, "run_kernel_trace.csv")
    dur = defaultdict(list)
    for r in trace:
        dur[r["Kernel_Name"]].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    counters = {}
    for d, cname in ((fetch_dir, "FETCH_SIZE"), (write_dir, "WRITE_SIZE")):
        vals = defaultdict(list)
        for r in rows(d, "run_counter_collection.csv"):
            if r["Counter_Name"] == cname:
                vals[r["Kernel_Name"]].append(float(r["Counter_Value"]))
        counters[cname] = vals
    gib_kib = float(1 << 20)
    copy_f = max(counters["FETCH_SIZE"]["__amd_rocclr_copyBuffer"])
    copy_w = max(counters["WRITE_SIZE"]["__amd_rocclr_copyBuffer"])
    f_scale, w_scale = gib_kib / copy_f, gib_kib / copy_w
    algo = {  # algorithmic bytes (flops for prefill) per launch of each workload
        "decode_0.6b": _decode_algo_bytes(256, 16, 100, 2048, 4096),
        "decode_fused_0.6b": _decode_algo_bytes(256, 16, 100, 2048, 4096, fused=True),
        "decode_8b": _decode_algo_bytes(128, 32, 1024, 32768, 20000),
        "append": 32522240,
    }
    # prefill: flops, and the algorithmic bytes beside them (prefill_bytes)
    qlens, klens, tables = prefill_workload()
    cq = [0] + list(itertools.accumulate(qlens))
    prefill_bytes_of = {}
    for key, kls, tbl in (("prefill", klens, tables), ("prefill_dense", qlens, None)):
        ck = [0] + list(itertools.accumulate(kls))
        algo[key] = prefill_flops(cq, ck, 16, D)
        prefill_bytes_of[key] = prefill_bytes(cq, ck, 16, 8, D, tbl, BS)
    algo.update(layer_algo_bytes(dict(T=LAYER_TOKENS, hq=16, hkv=8, H=1024, I=3072)))
    out_dir = ROOT / "profiles"
    out_dir.mkdir(exist_ok=True)
    merge_name = "kvp::decode_merge_kernel(kvp::DecodeParams)"
    for fname, prefix, key in PROFILE_KERNELS:
        names = [n for n in dur if n.startswith(prefix)]
        if not names:
            continue
        name = names[0]
        all_us = [x / 1e3 for x in dur[name]]
        d_us = all_us[len(all_us) // 3:]  # the first third covers the warm-up launches
        fetch = [x * f_scale * 1024 for x in counters["FETCH_SIZE"].get(name, [])]
        write = [x * w_scale * 1024 for x in counters["WRITE_SIZE"].get(name, [])]
        avg_us = statistics.mean(d_us)
        traffic = (statistics.mean(fetch) if fetch else 0) + (statistics.mean(write) if write else 0)
        lines = [f"# {fname}: `{name}`", "",
                 "Commands (from the repository root on the GPU host, `R=$PWD`, `OUT` a directory for the raw results):", "", "```"]
        lines += PROFILE_CMDS + ["```", ""]
        med_us = statistics.median(d_us)
        lines += [f"- dispatches: {len(all_us)}; over the last {len(d_us)} (after the warm-up launches) "
                  f"duration avg {avg_us:.2f} us, median {med_us:.2f} us, min {min(d_us):.2f}, "
                  f"max {max(d_us):.2f}"]
        if key.startswith("prefill"):
            nb = prefill_bytes_of[key]
            lines += [f"- algorithmic work: {algo[key]} flop (unmasked query-key pairs x 4 x Hq x D) "
                      f"-> {algo[key] / med_us / 1e6:.1f} TFLOP/s at the median duration "
                      f"({algo[key] / med_us / 1e6 / BF16_PEAK_TFLOPS * 100:.1f}% of 2.5 PFLOP/s dense bf16)",
                      f"- algorithmic bytes: {nb} (q and o once, each distinct key's K and V once) -> "
                      f"{nb / med_us / 1e3:.1f} GB/s at the median duration "
                      f"({nb / med_us / 1e3 / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s); intensity "
                      f"{algo[key] / nb:.0f} flop/B against the ridge point of 312 flop/B"]
        else:
            lines += [f"- algorithmic bytes: {algo[key]} -> {algo[key] / med_us / 1e3:.1f} GB/s at the median "
                      f"duration ({algo[key] / med_us / 1e3 / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)"]
        if key == "sample_t1":
            lines += ["- bound by the Philox noise arithmetic (ten rounds of two 32x32->64-bit products per "
                      "value, VALU), not by HBM: T = 1 on every row"]
        lines += [f"- FETCH_SIZE calibration: 1 GiB copy reads {copy_f:.1f} KiB -> scale {f_scale:.4f}; "
                  f"WRITE_SIZE: 1 GiB copy writes {copy_w:.1f} KiB -> scale {w_scale:.4f}",
                  f"- HBM traffic per dispatch (scaled): read {statistics.mean(fetch):.0f} B, "
                  f"write {statistics.mean(write):.0f} B, total {traffic:.0f} B"
                  + (f" = {traffic / (prefill_bytes_of[key] if key.startswith('prefill') else algo[key]):.4f} "
                     f"x algorithmic")]
        if key.startswith("decode") and merge_name in dur:
            m_us = [x / 1e3 for x in dur[merge_name]]
            m_us = m_us[len(m_us) // 3:]
            lines += [f"- the decode's split-combining `{merge_name}` (all decode workloads): "
                      f"median {statistics.median(m_us):.2f} us over {len(m_us)} dispatches"]
        (out_dir / f"{fname}.md").write_text("\n".join(lines) + "\n")
        if key == "decode_0.6b":
            (out_dir / "paged_decode_qwen3_0.6b_pmc.json").write_text(json.dumps(
                {"kernel": name, "traffic_bytes": int(round(traffic)), "fetch_scale": f_scale,
                 "write_scale": w_scale, "median_duration_us": med_us}, indent=1) + "\n")
        print(f"{fname}: median {med_us:.2f} us, traffic {traffic:.0f} B", flush=True)
    return 0


E2E_PROFILE_CMDS = [
    "cd /tmp && export TMPDIR=/tmp",
    "rocprofv3 --kernel-trace --stats --output-format csv -d $OUT/e2e_trace -o run -- python $R/bench.py --e2e-only",
    "python $R/bench.py --summarize-e2e $OUT/e2e_trace",
    "rocprofv3 --kernel-trace --stats --output-format csv -d $OUT/e2e_dropin -o run -- python $R/bench.py --e2e-only "
    "--e2e-caller dropin",
    "python $R/bench.py --summarize-e2e $OUT/e2e_dropin dropin",
]


def summarize_e2e(trace_dir: str, caller: str = "fused") -> int:
    """profiles/e2e_qwen3_0.6b.md (fused caller) or profiles/e2e_qwen3_0.6b_dropin.md:
    where the end-to-end generation spends GPU time, from the --stats output of rocprofv3
    over `bench.py --e2e-only [--e2e-caller dropin]`."""
    import csv

    with open(Path(trace_dir) / "run_kernel_stats.csv") as f:
        rows = list(csv.DictReader(f))
    total = sum(float(r["TotalDurationNs"]) for r in rows)

    def group(name):
        if name.startswith("Cijk") or name.startswith("Custom_Cijk"):
            return "hipBLASLt GEMMs (projections, MLP, LM head)"
        if "kvp::" in name:
            return name.replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")
        return "other (torch: embedding, copies, fills)"

    by = {}
    for r in rows:
        g = group(r["Name"])
        t, c = by.get(g, (0.0, 0))
        by[g] = (t + float(r["TotalDurationNs"]), c + int(r["Calls"]))
    title = "e2e_qwen3_0.6b" + ("" if caller == "fused" else "_" + caller)
    lines = [f"# {title}: GPU time of the end-to-end generation ({caller} attention caller), by kernel", "",
             "Commands (from the repository root on the GPU host, `R=$PWD`, `OUT` a directory for the raw results):", "", "```"]
    lines += E2E_PROFILE_CMDS + ["```", "",
                                 f"Total kernel time {total / 1e9:.3f} s (profiler overhead included; the "
                                 "untraced run's wall time is in bench.py's e2e_qwen3_0.6b field).", "",
                                 "| kernel | calls | total s | share | avg us |", "|---|---|---|---|---|"]
    for g, (t, c) in sorted(by.items(), key=lambda x: -x[1][0]):
        lines.append(f"| `{g}` | {c} | {t / 1e9:.3f} | {100 * t / total:.1f}% | {t / c / 1e3:.2f} |")
    out = ROOT / "profiles" / f"{title}.md"
    out.write_text("\n".join(lines) + "\n")
    print(f"wrote {out}", flush=True)
    return 0


def _decode_algo_bytes(B, hq, lo, hi, pool_blocks, seed=0, fused=False):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(lo, hi + 1, (B,), generator=g, dtype=torch.int32)
    return (fused_decode_bytes if fused else decode_bytes)(ctx.tolist(), hq, 8, D, BS)


# ----------------------------------------------------------------------------- end to end

def e2e_workload(num_seqs: int = 256, seed: int = 0):
    """Prompt / output lengths in the draw order of the reference's offline benchmark
    (benchs/bench.py:9-19: random.seed(0), per request a length in [100, 1024] then its
    ids, then every max_tokens in [100, 1024]), so the token counts match it
    (sum(max_tokens) = 133966 for 256 requests).  The ids themselves are then redrawn
    uniformly over the whole Qwen3 vocabulary (numpy, same seed)."""
    import random

    import numpy as np

    random.seed(seed)
    lengths = []
    for _ in range(num_seqs):
        n = random.randint(100, 1024)
        for _ in range(n):
            random.randint(0, 10000)
        lengths.append(n)
    max_tokens = [random.randint(100, 1024) for _ in range(num_seqs)]
    rng = np.random.default_rng(seed)
    prompts = [rng.integers(0, 151936, n).tolist() for n in lengths]
    return prompts, max_tokens


def bench_e2e(num_seqs: int = 256, caller: str = "fused", fused_decode: bool = True):
    """Offline generation with the Qwen3-0.6B architecture (random bf16 weights), greedy,
    ignore_eos, hipGraph decode, max_model_len 4096: output tok/s = sum(max_tokens) / wall.
    caller "dropin" runs the layers in the reference's order (q/k norm + RoPE, then
    Attention.forward appending through store_kvcache, dense prefill without a prefix)."""
    from kavor_amd.engine.llm_engine import LLM
    from kavor_amd.sampling_params import SamplingParams

    t0 = time.perf_counter()
    llm = LLM(None, enforce_eager=False, max_model_len=4096, seed=0, attention_caller=caller,
              fused_decode=fused_decode)
    init_s = time.perf_counter() - t0
    print(f"e2e: engine ready in {init_s:.1f}s ({llm.config.num_kvcache_blocks} pages, "
          f"{len(llm.model_runner.graphs)} graphs)", file=sys.stderr, flush=True)
    prompts, max_tokens = e2e_workload(num_seqs)
    sps = [SamplingParams(temperature=0.0, ignore_eos=True, max_tokens=m) for m in max_tokens]
    llm.generate([prompts[0][:16]], SamplingParams(temperature=0.0, max_tokens=4, ignore_eos=True))
    torch.cuda.synchronize()
    t = time.perf_counter()
    outs = llm.generate(prompts, sps)
    wall = time.perf_counter() - t
    print(f"e2e: generated {sum(max_tokens)} tokens in {wall:.2f}s", file=sys.stderr, flush=True)
    assert [len(o["token_ids"]) for o in outs] == max_tokens
    s = llm.throughput_summary()
    runner = llm.model_runner
    res = dict(
        output_tok_s=round(sum(max_tokens) / wall, 1),
        decode_tok_s=round(s["decode_tok_s"], 1),
        wall_s=round(wall, 3),
        output_tokens=sum(max_tokens), prompt_tokens=sum(len(p) for p in prompts),
        decode_steps=s["decode_steps"], decode_time_s=round(s["decode_time_s"], 3),
        prefill_steps=s["prefill_steps"], prefill_time_s=round(s["prefill_time_s"], 3),
        prefill_tok_s=round(s["prefill_tok_s"], 1),
        num_kvcache_blocks=llm.config.num_kvcache_blocks, graphs=len(runner.graphs),
        init_s=round(init_s, 2), capture_s=round(runner.timings["capture"], 2),
        workload=f"{num_seqs} requests, prompt U[100,1024] ids uniform over 151936, output U[100,1024], "
                 "greedy, ignore_eos, Qwen3-0.6B arch random bf16 weights, max_model_len 4096, "
                 f"hipGraph decode, block 256, {caller} attention caller"
                 + (", one-launch decode step" if caller == "fused" and fused_decode else ""),
    )
    llm.exit()
    del llm
    torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------ reference-design run

_EAGER_LEN: dict = {}


def _eager_attention_forward(self, positions: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
    """Qwen3Attention.forward with the paged KV path in plain PyTorch ops, the comparator
    standing in for the reference's design on this GPU: q/k RMSNorm and RoPE as separate
    steps, the append as an index-put into the pages, and attention as gather-then-softmax
    over the pages with explicit masks (bottom-right causal in prefill).  bf16 products
    take contiguous operands; scores and softmax are fp32.  Harness only: the product
    path never uses it."""
    import torch.nn.functional as F

    from kavor_amd.layers import fused
    from kavor_amd.utils.context import get_context

    T, Dh = hidden.shape[0], self.head_dim
    Hq, Hkv = self.num_heads, self.num_kv_heads
    G = Hq // Hkv
    qkv = F.linear(hidden, self.qkv_proj)
    q, k, v = qkv.split([self.q_size, self.kv_size, self.kv_size], dim=-1)
    q = fused.rms_norm(q.reshape(T, Hq, Dh), self.q_norm.weight, self.q_norm.eps)
    k = fused.rms_norm(k.reshape(T, Hkv, Dh), self.k_norm.weight, self.k_norm.eps)
    v = v.reshape(T, Hkv, Dh)
    cs = self.rope[positions.long()]
    cos, sin = cs[:, None, :Dh // 2], cs[:, None, Dh // 2:]

    def rope(x):
        x1, x2 = x.float().chunk(2, dim=-1)
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(torch.bfloat16)

    q, k = rope(q), rope(k)
    ctx = get_context()
    kc, vc = self.attn.k_cache[0], self.attn.v_cache[0]
    nb, bs = kc.shape[0], kc.shape[1]
    if kc.numel() > 0 and ctx.slot_mapping is not None:  # eager steps carry no padding slots
        sl = ctx.slot_mapping.long()
        kc[sl // bs, sl % bs] = k
        vc[sl // bs, sl % bs] = v
    scale = Dh ** -0.5
    if ctx.is_prefill:
        out = torch.empty(T, Hq, Dh, dtype=torch.bfloat16, device=q.device)
        cq, ck = ctx.cu_seqlens_q.tolist(), ctx.cu_seqlens_k.tolist()
        for i in range(len(cq) - 1):
            qlen, klen = cq[i + 1] - cq[i], ck[i + 1] - ck[i]
            if ctx.block_tables is not None:
                blocks = ctx.block_tables[i, :-(-klen // bs)].long()
                ks, vs = kc[blocks].reshape(-1, Hkv, Dh)[:klen], vc[blocks].reshape(-1, Hkv, Dh)[:klen]
            else:
                ks, vs = k[ck[i]:ck[i + 1]], v[ck[i]:ck[i + 1]]
            qh = q[cq[i]:cq[i + 1]].transpose(0, 1).float().contiguous()                     # [Hq, n, D]
            kt = ks.repeat_interleave(G, dim=1).permute(1, 2, 0).float().contiguous()       # [Hq, D, k]
            vh = vs.repeat_interleave(G, dim=1).transpose(0, 1).float().contiguous()        # [Hq, k, D]
            sc = torch.matmul(qh, kt) * scale
            r = torch.arange(qlen, device=q.device)[:, None]
            c = torch.arange(klen, device=q.device)[None, :]
            sc = sc.masked_fill(c > r + (klen - qlen), float("-inf"))
            out[cq[i]:cq[i + 1]] = torch.matmul(torch.softmax(sc, dim=-1), vh).transpose(0, 1).to(torch.bfloat16)
    else:
        # One host read per step, shared by the layers: the runner publishes a new Context
        # per step, and holding it keeps its identity from being reused.
        if _EAGER_LEN.get("ctx") is not ctx:
            _EAGER_LEN["ctx"] = ctx
            _EAGER_LEN["len"] = int(ctx.context_lens.max())
        W = -(-_EAGER_LEN["len"] // bs)
        L = W * bs
        bt = ctx.block_tables[:, :W].long().clamp(0, nb - 1)
        kt = kc[bt].reshape(T, L, Hkv, Dh).permute(0, 2, 3, 1).contiguous()   # [B, Hkv, D, L]
        vg = vc[bt].reshape(T, L, Hkv, Dh).transpose(1, 2).contiguous()        # [B, Hkv, L, D]
        sc = torch.matmul(q.reshape(T, Hkv, G, Dh), kt).float() * scale       # [B, Hkv, G, L]
        pad = torch.arange(L, device=q.device)[None, :] >= ctx.context_lens[:, None]
        sc = sc.masked_fill(pad[:, None, None, :], float("-inf"))
        # Positions past a sequence's length hold whatever the pages held (NaN bit
        # patterns included): a zero softmax weight times NaN is NaN, so clear them.
        vg.masked_fill_(pad[:, None, :, None], 0)
        out = torch.matmul(torch.softmax(sc, dim=-1).to(torch.bfloat16), vg).reshape(T, Hq, Dh)
    return F.linear(out.reshape(T, Hq * Dh), self.o_proj)


def bench_e2e_window(max_new: int = 32):
    """Decode throughput of the engine against the same engine with the PyTorch-eager
    attention path (the reference-design comparator), both eager (no graphs: the
    comparator's shapes change every step), on the end-to-end prompts with every
    request's output capped at `max_new` tokens."""
    from kavor_amd.engine import qwen3
    from kavor_amd.engine.llm_engine import LLM
    from kavor_amd.sampling_params import SamplingParams

    prompts, _ = e2e_workload()
    sps = SamplingParams(temperature=0.0, ignore_eos=True, max_tokens=max_new)
    res = {}
    native = qwen3.Qwen3Attention.forward
    for name, fwd in (("hip_path", native), ("torch_eager_attention", _eager_attention_forward)):
        qwen3.Qwen3Attention.forward = fwd
        try:
            llm = LLM(None, enforce_eager=True, max_model_len=4096, seed=0)
            llm.generate([prompts[0][:16]], SamplingParams(temperature=0.0, max_tokens=4, ignore_eos=True))
            torch.cuda.synchronize()
            t = time.perf_counter()
            llm.generate(prompts, sps)
            wall = time.perf_counter() - t
            sm = llm.throughput_summary()
            res[name] = dict(output_tok_s=round(len(prompts) * max_new / wall, 1),
                             decode_tok_s=round(sm["decode_tok_s"], 1), wall_s=round(wall, 3))
            llm.exit()
            del llm
        finally:
            qwen3.Qwen3Attention.forward = native
            _EAGER_LEN.clear()
        torch.cuda.empty_cache()
        print(f"e2e window {name}: {res[name]['decode_tok_s']} decode tok/s", file=sys.stderr, flush=True)
    res["decode_speedup"] = round(res["hip_path"]["decode_tok_s"] / res["torch_eager_attention"]["decode_tok_s"], 2)
    res["workload"] = (f"the 256 end-to-end prompts, {max_new} greedy output tokens each, both engines eager "
                       "(no graphs); comparator: q/k norm and RoPE as separate steps, index-put append, "
                       "gather + fp32 softmax attention in PyTorch")
    return res


# ----------------------------------------------------------------------------- main

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-extras", action="store_true", help="headline decode workload only")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end Qwen3-0.6B generation")
    ap.add_argument("--e2e-only", action="store_true", help="only the end-to-end generation (prints its JSON)")
    ap.add_argument("--e2e-seqs", type=int, default=256)
    ap.add_argument("--e2e-caller", choices=("fused", "dropin"), default="fused",
                    help="layer order of --e2e-only: the fused q/k kernel, or the reference's caller order")
    ap.add_argument("--summarize", nargs=3, metavar=("TRACE_DIR", "FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/*.md (and the decode traffic json) from the CSV output of "
                         "three rocprofv3 runs of --profile: --kernel-trace --stats, --pmc "
                         "FETCH_SIZE, --pmc WRITE_SIZE")
    ap.add_argument("--profile", action="store_true",
                    help="the default run's kernel launches without the CPU baseline and the engine, "
                         "for rocprofv3; starts with plain 1 GiB device copies used to calibrate "
                         "FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="only the prefix-cached prefill launches (30), for rocprofv3 --pmc passes")
    ap.add_argument("--summarize-prefill-pmc", nargs=3, metavar=("PASS_A_DIR", "PASS_B_DIR", "PASS_C_DIR"),
                    help="write profiles/varlen_prefill_prefix_32seq_pmc.md from the three --pmc passes")
    ap.add_argument("--summarize-e2e", nargs="+", metavar="TRACE_DIR [CALLER]",
                    help="write profiles/e2e_qwen3_0.6b.md from rocprofv3 --stats over --e2e-only")
    args = ap.parse_args()
    if args.summarize:
        return summarize_profiles(*args.summarize)
    if args.summarize_e2e:
        return summarize_e2e(*args.summarize_e2e)
    if args.summarize_prefill_pmc:
        return summarize_prefill_pmc(*args.summarize_prefill_pmc)
    if args.gpus != 1:
        print(f"bench.py measures one GPU's paged KV-cache kernels; --gpus {args.gpus} is not "
              "supported (the path shards by kv head with no exchange inside attention).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    from kavor_amd._lib import lib

    lib()
    if args.profile:
        return profile_run(dev, args.steps, args.warmup)
    if args.profile_prefill:
        bench_prefill(dev, 20, 10)
        torch.cuda.synchronize()
        print("prefill profile run done", flush=True)
        return 0
    if args.e2e_only:
        print(json.dumps({"e2e_qwen3_0.6b": bench_e2e(args.e2e_seqs, args.e2e_caller)}), flush=True)
        return 0

    # The headline is timed first: after the extra workloads (seconds of full-power GPU
    # work) the same decode reads about 3% slower until the part has idled for a while.
    inp, dec = bench_decode(dev, args.steps, args.warmup, "qwen3_0.6b")
    extras = {}
    if not args.no_extras:
        extras.update(run_extras(dev, args.steps, args.warmup, cpu_baseline=not args.no_cpu_baseline))
    cpu = None if args.no_cpu_baseline else cpu_baseline_decode(inp)
    if not args.no_cpu_baseline and not args.no_extras:
        extras["kv_append"]["cpu_baseline"] = cpu_baseline_append()
        extras["varlen_prefill"]["cpu_baseline"] = cpu_baseline_prefill()
    if not args.no_e2e:
        del inp
        torch.cuda.empty_cache()
        extras["e2e_qwen3_0.6b"] = bench_e2e(args.e2e_seqs)
        d = bench_e2e(args.e2e_seqs, fused_decode=False)
        extras["e2e_qwen3_0.6b"]["separate_decode_launches"] = {
            k: d[k] for k in ("output_tok_s", "decode_tok_s", "wall_s", "workload")}
        d = bench_e2e(args.e2e_seqs, caller="dropin")
        extras["e2e_qwen3_0.6b"]["dropin"] = {k: d[k] for k in ("output_tok_s", "decode_tok_s", "wall_s",
                                                               "prefill_tok_s", "workload")}
        extras["e2e_qwen3_0.6b"]["reference_design"] = bench_e2e_window()
        if not args.no_cpu_baseline:
            extras["e2e_qwen3_0.6b"]["cpu_baseline"] = cpu_baseline_e2e()

    gbs = dec["gbs"]
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "paged decode, Qwen3-0.6B layer: B=256, 16q/8kv heads, head_dim 128, "
                               "ctx U[100,2048], block 256, pool 4096 blocks",
                   "bytes_per_step": dec["bytes"]},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic("paged_decode_qwen3_0.6b_pmc")},
        "cpu_baseline": cpu,
        **extras,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
