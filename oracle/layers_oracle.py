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

Pinned by tests/test_oracle_layers.py against closed forms (a rotation by the Qwen3
frequencies is norm preserving and equals complex multiplication; RMSNorm of a scaled
row is scale invariant; SiLU(0) = 0 and SiLU(x) -> x) and by the reference's own test
tolerances (tests/test_fused_kernels.py:40-90: rtol = atol = 2e-2 against these forms).
"""

from __future__ import annotations

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
