"""Pins of the layer oracle (oracle/layers_oracle.py) against closed forms (CPU).

Each check is chosen so that a plausible slip fails it: a rotation by the wrong
frequencies or a swapped sin sign breaks the complex-multiplication identity, a wrong
RMS denominator breaks scale invariance and the unit-RMS identity, a dropped fp32
upcast of the residual sum breaks the bf16-rounded residual, a tie broken towards the
last index breaks the first-occurrence rule.
"""

import math

import torch

from oracle.layers_oracle import (add_rms_norm, apply_rope, greedy, qk_norm_rope, rms_norm,
                                  rope_table, silu_and_mul)


def test_rms_norm_closed_form_and_scale_invariance():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 256, generator=g, dtype=torch.float64)
    w = torch.ones(256, dtype=torch.float64)
    y = rms_norm(x, w, 0.0)
    # unit RMS, scale invariance (the oracle computes in fp32)
    torch.testing.assert_close(y.square().mean(-1), torch.ones(5, dtype=torch.float64), atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(rms_norm(7.0 * x, w, 0.0), y, atol=1e-6, rtol=1e-6)
    xb = torch.randn(5, 256, generator=g).to(torch.bfloat16)
    wb = (1 + 0.1 * torch.randn(256, generator=g)).to(torch.bfloat16)
    xd = xb.double()
    want = (xd / torch.sqrt(xd.square().mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16).double() * wb.double()
    torch.testing.assert_close(rms_norm(xb, wb, 1e-6).double(), want, atol=2e-2, rtol=1e-2)


def test_add_rms_norm_rounds_the_fp32_sum_once():
    x = torch.tensor([[1.0, 2.0 ** -9, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]], dtype=torch.bfloat16)
    r = torch.tensor([[2.0 ** -9, 1.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]], dtype=torch.bfloat16)
    w = torch.ones(8, dtype=torch.bfloat16)
    _, res = add_rms_norm(x, r, w, 1e-6)
    # bf16 keeps 7 fraction bits: 1 + 2^-9 is under half an ulp above 1 and rounds to 1
    assert res[0, 0].item() == 1.0 and res[0, 1].item() == 1.0
    s = x.double() + r.double()
    y, _ = add_rms_norm(x, r, w, 1e-6)
    want = s / torch.sqrt(s.square().mean(-1, keepdim=True) + 1e-6)
    torch.testing.assert_close(y.double(), want, atol=1e-2, rtol=1e-2)


def test_rope_table_and_rotation():
    D, base = 128, 1e6
    table = rope_table(D, 64, base)
    i = torch.arange(D // 2, dtype=torch.float64)
    for p in (0, 1, 37, 63):
        ang = p * base ** (-2 * i / D)
        torch.testing.assert_close(table[p, :D // 2].double(), torch.cos(ang), atol=5e-6, rtol=0)
        torch.testing.assert_close(table[p, D // 2:].double(), torch.sin(ang), atol=5e-6, rtol=0)
    x = torch.randn(3, 2, D, dtype=torch.float32)
    pos = torch.tensor([0, 5, 63])
    cos, sin = table[pos].unsqueeze(1).chunk(2, dim=-1)
    y = apply_rope(x, cos, sin)
    torch.testing.assert_close(y[0], x[0])
    torch.testing.assert_close(y.norm(dim=-1), x.norm(dim=-1))
    z = torch.complex(x[1, 0, :D // 2].double(), x[1, 0, D // 2:].double())
    zr = z * torch.exp(1j * 5 * base ** (-2 * i / D))
    torch.testing.assert_close(y[1, 0, :D // 2].double(), zr.real, atol=1e-5, rtol=0)
    torch.testing.assert_close(y[1, 0, D // 2:].double(), zr.imag, atol=1e-5, rtol=0)


def test_qk_norm_rope_splits_heads_in_qwen3_order():
    D, hq, hkv = 128, 4, 2
    g = torch.Generator().manual_seed(1)
    qkv = torch.randn(3, (hq + 2 * hkv) * D, generator=g).to(torch.bfloat16)
    table = rope_table(D, 16, 1e6)
    ones = torch.ones(D, dtype=torch.bfloat16)
    q, k, v = qk_norm_rope(qkv, torch.tensor([0, 0, 0]), table, ones, ones, 1e-6, hq, hkv)
    assert torch.equal(v, qkv[:, (hq + hkv) * D:].reshape(3, hkv, D))
    # position 0: RoPE is the identity, so q / k are the normalised heads
    torch.testing.assert_close(q, rms_norm(qkv[:, :hq * D].reshape(3, hq, D), ones, 1e-6))
    torch.testing.assert_close(k, rms_norm(qkv[:, hq * D:(hq + hkv) * D].reshape(3, hkv, D), ones, 1e-6))


def test_silu_and_mul_closed_form():
    g = torch.tensor([[0.0, 1.0, -1.0, 20.0]], dtype=torch.float64)
    u = torch.tensor([[3.0, 2.0, 2.0, 0.5]], dtype=torch.float64)
    out = silu_and_mul(torch.cat([g, u], dim=-1))
    want = [0.0, 2.0 / (1 + math.exp(-1)), -2.0 / (1 + math.exp(1)), 20.0 * 0.5 / (1 + math.exp(-20))]
    torch.testing.assert_close(out[0], torch.tensor(want, dtype=torch.float64))


def test_greedy_first_index_on_ties():
    logits = torch.tensor([[1.0, 3.0, 3.0, 2.0], [5.0, 5.0, 5.0, 5.0]], dtype=torch.bfloat16)
    assert greedy(logits).tolist() == [1, 0]
