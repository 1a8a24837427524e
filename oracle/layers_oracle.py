"""Oracle for the layer work around the paged KV path (test infrastructure only).

Plain PyTorch restatements of the reference's eager formulas, used by tests/ to check
the fused HIP kernels and the engine; nothing in the product imports this module.

  rms_norm, add_rms_norm   kavor/layers/layernorm.py:260-284 (the eager formula in
                           add_rms_forward's docstring and rms_forward's fallback,
                           :247-252): fp32 statistics, bf16 rounding, then * weight in bf16
  rope_table, apply_rope   kavor/layers/rotary_embedding.py:56-66, 84-101 (neox pairing
                           (x_i, x_{i+D/2}), fp32 rotation, one rounding)
  silu_and_mul             kavor/layers/activation.py:6-11 (torch.compile keeps fp32
                           intermediates: one rounding at the end)
  greedy                   kavor/layers/sampler.py:34-44 at T = 0: argmax, first index on ties
  philox4x32_10, uniform,  kavor/layers/sampler.py:7-45 at T > 0: u = tl.rand(seed, i + r * V),
  gumbel_scores, sample    score = logit / T - log(-log(u)), the first index of the largest
                           score.  tl.rand is Triton's (triton/language/random.py, 3.6.0 here):
                           the first word of Philox4x32-10 (Salmon et al., SC 2011) for
                           counter (offset, 0, 0, 0) and key (seed low, seed high), as int32 x,
                           x < 0 folded to -x - 1, times 4.6566127342e-10

The sampling functions are pinned by tests/test_oracle_layers.py against the published
Philox4x32-10 known-answer vectors (Random123's kat_vectors), against tl.rand words and
floats written by Triton's own interpreter (tests/golden/make_philox.py), and by a
chi-square test of the sampled frequencies against softmax(logits / T).  The rest is
pinned by tests/test_oracle_layers.py against closed forms (a rotation by the Qwen3
frequencies is norm preserving and equals complex multiplication; RMSNorm of a scaled
row is scale invariant; SiLU(0) = 0 and SiLU(x) -> x) and by the reference's own test
tolerances (tests/test_fused_kernels.py:40-90: rtol = atol = 2e-2 against these forms).
"""

from __future__ import annotations

import numpy as np
import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    xf = xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)
    return xf.to(x.dtype) * weight


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    xf = x.float() + residual.float()
    residual = xf.to(x.dtype)
    xf = xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)
    return xf.to(x.dtype) * weight, residual


def rope_table(head_dim: int, max_position: int, base: float, device="cpu") -> torch.Tensor:
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    t = torch.arange(max_position, dtype=torch.float32, device=device)
    freqs = torch.outer(t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [T, H, D] rotated by per-token cos/sin [T, 1, D/2]."""
    x1, x2 = x.float().chunk(2, dim=-1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)


def qk_norm_rope(qkv: torch.Tensor, positions: torch.Tensor, table: torch.Tensor,
                 q_w: torch.Tensor, k_w: torch.Tensor, eps: float, hq: int, hkv: int):
    """q/k RMSNorm then RoPE of the fused qkv rows (qwen3.py:80-89); returns q, k, v."""
    D = table.shape[1]
    T = qkv.shape[0]
    q, k, v = qkv.split([hq * D, hkv * D, hkv * D], dim=-1)
    q = rms_norm(q.reshape(T, hq, D), q_w, eps)
    k = rms_norm(k.reshape(T, hkv, D), k_w, eps)
    cos, sin = table[positions.long()].unsqueeze(1).chunk(2, dim=-1)
    return apply_rope(q, cos, sin), apply_rope(k, cos, sin), v.reshape(T, hkv, D)


def silu_and_mul(gate_up: torch.Tensor) -> torch.Tensor:
    g, u = gate_up.float().chunk(2, dim=-1)
    return (g * torch.sigmoid(g) * u).to(gate_up.dtype)


def greedy(logits: torch.Tensor) -> torch.Tensor:
    return logits.float().argmax(dim=-1)


# ----------------------------------------------------------------------- sampling (T > 0)

_PHILOX_MUL = (np.uint64(0xD2511F53), np.uint64(0xCD9E8D57))
_PHILOX_WEYL = (np.uint32(0x9E3779B9), np.uint32(0xBB67AE85))


def philox4x32_10(c0, c1, c2, c3, k0, k1):
    """Philox4x32 with 10 rounds, elementwise over uint32 arrays (counter words c0..c3,
    key words k0, k1); returns the four output words."""
    c = [np.asarray(x, dtype=np.uint32).astype(np.uint64) for x in (c0, c1, c2, c3)]
    k = [np.asarray(x, dtype=np.uint32).copy() for x in (k0, k1)]
    lo = np.uint64(0xFFFFFFFF)
    for _ in range(10):
        pa = _PHILOX_MUL[0] * c[0]
        pb = _PHILOX_MUL[1] * c[2]
        n0 = (pb >> np.uint64(32)) ^ c[1] ^ k[0].astype(np.uint64)
        n2 = (pa >> np.uint64(32)) ^ c[3] ^ k[1].astype(np.uint64)
        c = [n0 & lo, pb & lo, n2 & lo, pa & lo]
        k = [k[0] + _PHILOX_WEYL[0], k[1] + _PHILOX_WEYL[1]]
    return tuple(x.astype(np.uint32) for x in c)


def uniform(word) -> np.ndarray:
    """Triton's uint_to_uniform_float for 32-bit words: float32 in [0, 1)."""
    x = np.asarray(word, dtype=np.uint32).view(np.int32).astype(np.int64)
    x = np.where(x < 0, -x - 1, x)
    return x.astype(np.float32) * np.float32(4.6566127342e-10)


def tl_rand(seed: int, offsets) -> np.ndarray:
    """tl.rand(seed, offsets) for an int32 seed and 32-bit offsets."""
    off = np.asarray(offsets, dtype=np.int64).astype(np.uint32)
    s64 = np.int64(seed).astype(np.uint64)
    k0 = np.full(off.shape, np.uint32(s64 & np.uint64(0xFFFFFFFF)), dtype=np.uint32)
    k1 = np.full(off.shape, np.uint32(s64 >> np.uint64(32)), dtype=np.uint32)
    z = np.zeros(off.shape, dtype=np.uint32)
    return uniform(philox4x32_10(off, z, z, z, k0, k1)[0])


def gumbel_scores(logits: torch.Tensor, temperatures, seed: int) -> np.ndarray:
    """[B, V] float32 scores: logit / T - log(-log(u)) for rows with T > 0, the logit
    otherwise; u = tl.rand(seed, i + r * V) (offsets wrap at 2^32, as int32 arithmetic)."""
    lg = logits.float().cpu().numpy().astype(np.float32)
    B, V = lg.shape
    t = np.asarray(temperatures, dtype=np.float32).reshape(-1)[:B]
    out = lg.copy()
    rows = np.flatnonzero(t > 0)
    step = max(1, (1 << 22) // max(V, 1))  # rows per block: about 4M draws at a time
    with np.errstate(divide="ignore", invalid="ignore"):
        for b0 in range(0, rows.size, step):
            r = rows[b0:b0 + step]
            off = (r[:, None].astype(np.int64) * V + np.arange(V, dtype=np.int64)[None, :]) % (1 << 32)
            g = -np.log(-np.log(tl_rand(seed, off)))
            out[r] = lg[r] / t[r][:, None] + g.astype(np.float32)
    return out


def first_argmax(scores: np.ndarray) -> np.ndarray:
    """Per row, the first index of the largest score, a NaN counting as largest."""
    s = np.asarray(scores, dtype=np.float32)
    nan = np.isnan(s)
    idx = np.where(nan, -np.inf, s).argmax(axis=1)  # numpy keeps the first maximum
    return np.where(nan.any(axis=1), nan.argmax(axis=1), idx).astype(np.int64)


def sample(logits: torch.Tensor, temperatures, seed: int) -> np.ndarray:
    return first_argmax(gumbel_scores(logits, temperatures, seed))
