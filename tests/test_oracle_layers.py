"""Pins of the layer oracle (oracle/layers_oracle.py) against closed forms (CPU).

Each check is chosen so that a plausible slip fails it: a rotation by the wrong
frequencies or a swapped sin sign breaks the complex-multiplication identity, a wrong
RMS denominator breaks scale invariance and the unit-RMS identity, a dropped fp32
upcast of the residual sum breaks the bf16-rounded residual, a tie broken towards the
last index breaks the first-occurrence rule.  The sampling oracle is pinned by the
published Philox4x32-10 known answers, by Triton's own tl.randint / tl.rand outputs
(tests/golden/philox_triton.npz), and by the sampled frequencies: a wrong temperature or
a sign slip in the Gumbel noise moves them away from softmax(logits / T).
"""

import math
from pathlib import Path

import numpy as np
import torch

from oracle.layers_oracle import (add_rms_norm, apply_rope, first_argmax, greedy, gumbel_scores, philox4x32_10,
                                  qk_norm_rope, rms_norm, rope_table, sample, silu_and_mul, tl_rand, uniform)

GOLDEN = Path(__file__).resolve().parent / "golden"


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


# Random123's kat_vectors for philox4x32 with 10 rounds: counter, key, output.
PHILOX_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


def test_philox_known_answers():
    for ctr, key, want in PHILOX_KAT:
        got = philox4x32_10(*[np.array([x], dtype=np.uint32) for x in ctr + key])
        assert tuple(int(w[0]) for w in got) == want


def test_tl_rand_matches_triton_vectors():
    d = np.load(GOLDEN / "philox_triton.npz")
    for i, seed in enumerate(d["seeds"]):
        off = d["offsets"].astype(np.int64)
        u = tl_rand(int(seed), off)
        assert np.array_equal(u, d["floats"][i]), int(seed)
        assert np.array_equal(uniform(d["words"][i]), d["floats"][i])


def test_uniform_edges():
    w = np.array([0, 0xFFFFFFFF, 0x7FFFFFFF, 0x80000000, 1, 0xFFFFFFFE], dtype=np.uint32)
    u = uniform(w)
    assert u[0] == 0 and u[1] == 0          # 0 and -1 fold onto 0
    assert u[2] == u[3] and u[2] < 1.0       # the largest magnitude stays below 1
    assert u[4] == u[5] > 0


def _chi2(counts: np.ndarray, probs: np.ndarray) -> float:
    expect = counts.sum() * probs
    return float(((counts - expect) ** 2 / expect).sum())


def test_sampled_frequencies_follow_softmax_over_temperature():
    """20,000 rows of the same 6 logits, each row its own noise (offsets r * V + i): the
    counts fit softmax(logits / T) (chi-square, 5 degrees of freedom, p = 1e-4 bound 25.7)
    and do not fit the same logits at T = 1 or with the noise's sign flipped."""
    logits = torch.tensor([0.0, 1.0, 2.0, -1.0, 0.5, 3.0]).to(torch.bfloat16)
    T, rows, seed = 0.8, 20000, 1234
    lg = logits.float().repeat(rows, 1)
    idx = sample(lg, np.full(rows, T, dtype=np.float32), seed)
    counts = np.bincount(idx, minlength=6).astype(np.float64)
    p = torch.softmax(logits.float() / T, 0).double().numpy()
    assert _chi2(counts, p) < 25.7
    assert _chi2(counts, torch.softmax(logits.float(), 0).double().numpy()) > 200
    flipped = first_argmax(2 * lg.numpy() / T - gumbel_scores(lg, np.full(rows, T, dtype=np.float32), seed))
    assert _chi2(np.bincount(flipped, minlength=6).astype(np.float64), p) > 200


def test_sampling_at_temperature_zero_is_greedy_and_rows_draw_their_own_noise():
    g = torch.Generator().manual_seed(5)
    lg = torch.randn(6, 1000, generator=g).to(torch.bfloat16)
    temps = np.array([0.0, 1.0, -1.0, float("nan"), 1.0, 0.0], dtype=np.float32)
    idx = sample(lg, temps, 9)
    greedy_rows = [0, 2, 3, 5]
    assert np.array_equal(idx[greedy_rows], greedy(lg)[greedy_rows].numpy())
    # rows 1 and 4 hold different logits but also different noise: their scores differ
    # from the same row's scores under another seed
    s9 = gumbel_scores(lg, temps, 9)
    s10 = gumbel_scores(lg, temps, 10)
    assert not np.array_equal(s9[1], s10[1])
    assert np.array_equal(s9[0], lg[0].float().numpy())
