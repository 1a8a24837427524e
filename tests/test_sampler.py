"""The device sampler (kvp_sample_bf16, kavor/layers/sampler.py:7-66) against the oracle.

Rows with a temperature above 0 draw argmax(logits / T - log(-log(u))) with u the
reference's noise stream (Triton's tl.rand(seed, i + r * V)); the others take the greedy
index.  The oracle restates the stream bit for bit (pinned in test_oracle_layers.py), so
the sampled indices must equal the oracle's; a mismatch is only allowed where the
oracle's two candidate scores agree to float32 rounding (a tie the kernel's logarithm may
break the other way).  Also: greedy rows equal kvp_argmax_bf16, split and whole rows
agree, the seed advances once per call, the frequencies follow softmax(logits / T), and
a captured graph draws new noise on every replay.
"""

import numpy as np
import pytest
import torch

from kavor_amd.layers.fused import argmax_workspace, greedy_argmax, sample
from oracle import layers_oracle as lref

pytestmark = pytest.mark.gpu


def _check_against_oracle(logits_host, temps_host, seed_used, got):
    scores = lref.gumbel_scores(logits_host, temps_host, seed_used)
    want = lref.first_argmax(scores)
    got = np.asarray(got)
    for r in np.flatnonzero(got != want):
        a, b = scores[r, got[r]], scores[r, want[r]]
        assert abs(a - b) <= 4e-7 * max(1.0, abs(b)), (r, got[r], want[r], a, b)
    assert (got == want).mean() >= 0.99


def _temps(rows, g):
    base = [0.0, 0.7, 1.0, 1e3, 0.05, float("nan"), -1.0, 2.5]
    return torch.tensor([base[i % len(base)] for i in range(rows)], dtype=torch.float32)


@pytest.mark.parametrize("rows,vocab", [(1, 151936), (7, 151936 + 5), (64, 151936), (191, 4096), (256, 4096),
                                        (256, 151936 // 8), (5, 13), (9, 8)])
def test_sample_matches_oracle(cuda_device, rows, vocab):
    g = torch.Generator().manual_seed(rows * 1000 + vocab)
    logits = (torch.randn(rows, vocab, generator=g) * 3).to(torch.bfloat16)
    temps = _temps(rows, g)
    seed = torch.tensor([41 + rows], dtype=torch.int32, device=cuda_device)
    # rows padded to a multiple of 8 elements (the kernel's row-stride rule); the noise
    # offsets are r * vocab + i whatever the stride
    buf = torch.zeros(rows, (vocab + 7) // 8 * 8 + 8, dtype=torch.bfloat16)
    buf[:, :vocab] = logits
    got = sample(buf.to(cuda_device)[:, :vocab], temps.to(cuda_device), seed).cpu()
    assert seed.item() == 42 + rows                      # advanced once, before drawing
    _check_against_oracle(logits, temps.numpy(), 42 + rows, got.numpy())
    greedy_rows = [r for r in range(rows) if not temps[r] > 0]
    if greedy_rows:
        assert torch.equal(got[greedy_rows], lref.greedy(logits)[greedy_rows])


def test_sample_split_rows_equal_whole_rows_and_greedy_kernel(cuda_device):
    from kavor_amd._lib import check, lib

    rows, V = 40, 151936
    g = torch.Generator().manual_seed(3)
    logits = (torch.randn(rows, V, generator=g) * 2).to(torch.bfloat16).to(cuda_device)
    logits[5, 77] = float("nan")                          # a NaN score counts as largest
    temps = _temps(rows, g).to(cuda_device)
    seed = torch.tensor([7], dtype=torch.int32, device=cuda_device)
    split = sample(logits, temps, seed.clone()).cpu()     # draws with seed 8
    whole = torch.empty(rows, dtype=torch.int64, device=cuda_device)
    s8 = torch.tensor([8], dtype=torch.int32, device=cuda_device)
    rc = lib().kvp_sample_bf16(logits.data_ptr(), logits.stride(0), rows, V, temps.data_ptr(), s8.data_ptr(),
                               whole.data_ptr(), None, 0, torch.cuda.current_stream(cuda_device).cuda_stream)
    check("kvp_sample_bf16", rc)
    assert torch.equal(split, whole.cpu())
    assert split[5].item() == 77
    zero = torch.zeros(rows, dtype=torch.float32, device=cuda_device)
    assert torch.equal(sample(logits, zero, seed).cpu(), greedy_argmax(logits).cpu())


def test_sampled_frequencies_follow_softmax(cuda_device):
    """16,384 rows of the same 16 logits: chi-square of the counts against
    softmax(logits / T) (15 degrees of freedom, p = 1e-4 bound 42.6)."""
    logits = torch.linspace(-2.0, 2.5, 16).to(torch.bfloat16)
    rows, T = 16384, 1.3
    x = logits.repeat(rows, 1).to(cuda_device)
    temps = torch.full((rows,), T, dtype=torch.float32, device=cuda_device)
    seed = torch.tensor([100], dtype=torch.int32, device=cuda_device)
    counts = np.bincount(sample(x, temps, seed).cpu().numpy(), minlength=16).astype(np.float64)
    p = torch.softmax(logits.float() / T, 0).double().numpy()
    expect = rows * p
    assert float(((counts - expect) ** 2 / expect).sum()) < 42.6


def test_sample_in_a_graph_draws_new_noise_each_replay(cuda_device):
    rows, V = 16, 151936
    g = torch.Generator().manual_seed(11)
    logits = (torch.randn(rows, V, generator=g) * 3).to(torch.bfloat16)
    temps = torch.full((rows,), 1.0, dtype=torch.float32)
    temps[3] = 0.0
    dl, dt = logits.to(cuda_device), temps.to(cuda_device)
    seed = torch.tensor([500], dtype=torch.int32, device=cuda_device)
    out = torch.empty(rows, dtype=torch.int64, device=cuda_device)
    argmax_workspace(cuda_device)
    sample(dl, dt, seed, out=out)                         # eager: seed 501
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sample(dl, dt, seed, out=out)
    seed.fill_(600)
    draws = []
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        draws.append(out.cpu().numpy().copy())
        torch.cuda.synchronize()
    assert seed.item() == 603
    for k, got in enumerate(draws):
        _check_against_oracle(logits, temps.numpy(), 601 + k, got)
    assert not np.array_equal(draws[0], draws[1])
