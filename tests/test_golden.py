"""The oracle still reproduces the committed golden fixtures (CPU)."""

from pathlib import Path

import numpy as np
import torch

from oracle import kvpath_oracle as ref

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.astype(np.uint16).view(np.int16)).view(torch.bfloat16)


def test_golden_append():
    f = load("append_small")
    nb, bs, hkv, d = (int(x) for x in f["dims"])
    pool = torch.from_numpy(f["pool_before"].copy())
    kc, vc = ref.page_views(pool, bs, hkv, d)
    ref.kv_append(f["key"], f["value"], ref.bf16_bits(kc), ref.bf16_bits(vc), f["slot_mapping"])
    assert np.array_equal(pool.numpy(), f["pool_after"])


def test_golden_decode():
    f = load("decode_small")
    out = ref.paged_decode(bf16(f["q"]), bf16(f["k_cache"]), bf16(f["v_cache"]),
                           torch.from_numpy(f["block_tables"]), torch.from_numpy(f["context_lens"]),
                           float(f["scale"]), dtype=torch.float64)
    assert np.array_equal(out.numpy(), f["out"])


def test_golden_prefill():
    f = load("prefill_small")
    out = ref.varlen_prefill(bf16(f["q"]), bf16(f["k_cache"]), bf16(f["v_cache"]),
                             torch.from_numpy(f["cu_seqlens_q"]), torch.from_numpy(f["cu_seqlens_k"]),
                             float(f["scale"]), block_tables=torch.from_numpy(f["block_tables"]),
                             dtype=torch.float64)
    np.testing.assert_allclose(out.numpy(), f["out"], rtol=0, atol=1e-12)
