"""Writes the small golden fixtures under tests/golden/ (run from the repository root:
``python tests/golden/make_golden.py``).

Inputs are drawn from fixed seeds; expected outputs come from the pinned oracle
(oracle/kvpath_oracle.py, float64 for attention, a bit copy for the append) and, where a
closed form exists, are the closed form itself (the one-token decode rows return their V
row).  bf16 data is stored as its uint16 bit pattern.  The reference's own tests hold no
vectors for this path, so these fixtures freeze the oracle's answers: tests check that
the oracle still reproduces them and that the HIP kernels match them.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import kvpath_oracle as ref  # noqa: E402
from tests.helpers import gen, randn_bf16, interleaved_pool, random_block_tables  # noqa: E402


def u16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def make_append() -> dict:
    """Engine page layout (K/V interleaved pages), Qwen3-style strided value rows,
    padding slots in the middle and at the tail."""
    g = gen(101)
    nb, bs, hkv, d, n = 6, 64, 2, 128, 40
    pool, kc, vc = interleaved_pool(nb, bs, hkv, d, g)
    key = randn_bf16((n, hkv, d), g)
    wide = randn_bf16((n, 4 * hkv * d), g)
    value = wide[:, 3 * hkv * d:].view(n, hkv, d)
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int32)
    slots[[3, 17, 38, 39]] = -1
    pool_before = pool.clone()
    ref.kv_append(ref.bf16_bits(key), ref.bf16_bits(value), ref.bf16_bits(kc), ref.bf16_bits(vc),
                  slots.numpy())
    return dict(key=u16(key), value=u16(value), slot_mapping=slots.numpy(),
                pool_before=pool_before.numpy(), pool_after=pool.numpy(),
                dims=np.array([nb, bs, hkv, d]))


def make_decode() -> dict:
    """GQA 2, block size 64, contexts spanning 1, 2 and 3 blocks plus a one-token and an
    empty context (closed forms: V row, zeros)."""
    g = gen(102)
    nb, bs, hkv, hq, d = 12, 64, 1, 2, 128
    ctx = [1, 64, 65, 150, 0, 129]
    kc, vc = randn_bf16((nb, bs, hkv, d), g), randn_bf16((nb, bs, hkv, d), g)
    bt = random_block_tables(ctx, bs, nb, g, width=3)
    q = randn_bf16((len(ctx), hq, d), g)
    scale = 128 ** -0.5
    out = ref.paged_decode(q, kc, vc, bt, torch.tensor(ctx), scale, dtype=torch.float64)
    # closed form for the one-token row: each query head returns its kv head's V row
    one = vc[int(bt[0, 0]), 0, 0].double()
    assert torch.equal(out[0, 0], one) and torch.equal(out[0, 1], one)
    return dict(q=u16(q), k_cache=u16(kc), v_cache=u16(vc), block_tables=bt.numpy(),
                context_lens=np.array(ctx, dtype=np.int32), scale=np.array(scale),
                out=out.numpy())


def make_prefill() -> dict:
    """Paged prefill with cached prefixes (one block-aligned, one not, one empty) and GQA 2."""
    g = gen(103)
    nb, bs, hkv, hq, d = 16, 64, 1, 2, 128
    qlens, prefix = [70, 5, 33], [128, 37, 0]
    klens = [a + b for a, b in zip(qlens, prefix)]
    kc, vc = randn_bf16((nb, bs, hkv, d), g), randn_bf16((nb, bs, hkv, d), g)
    bt = random_block_tables(klens, bs, nb, g, width=4)
    q = randn_bf16((sum(qlens), hq, d), g)
    cq = torch.tensor(np.cumsum([0] + qlens), dtype=torch.int32)
    ck = torch.tensor(np.cumsum([0] + klens), dtype=torch.int32)
    scale = 128 ** -0.5
    out = ref.varlen_prefill(q, kc, vc, cq, ck, scale, block_tables=bt, dtype=torch.float64)
    return dict(q=u16(q), k_cache=u16(kc), v_cache=u16(vc), block_tables=bt.numpy(),
                cu_seqlens_q=cq.numpy(), cu_seqlens_k=ck.numpy(), scale=np.array(scale),
                out=out.numpy())


def main() -> None:
    for name, fn in (("append_small", make_append), ("decode_small", make_decode),
                     ("prefill_small", make_prefill)):
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **fn())
        print(path, path.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
