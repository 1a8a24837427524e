"""Token sampler (kavor/layers/sampler.py:7-66).

Every call advances a device seed by one and draws with it, as the reference's
Sampler.forward does, so that a captured graph draws new noise on each replay.  Rows
with a temperature above 0 take a Gumbel-max sample of softmax(logits / T) from the
reference's noise stream (Philox4x32-10 words at offsets i + r * V, as Triton's tl.rand
draws them); the others take the greedy index (first on ties).  Both run as one HIP
kernel, kvp_sample_bf16; an all-greedy batch outside a graph takes the argmax kernel
(kvp_argmax_bf16) directly.
"""

from __future__ import annotations

import torch

from kavor_amd.layers.fused import greedy_argmax, sample


class Sampler:

    def __init__(self, device):
        self.seed = torch.zeros(1, dtype=torch.int32, device=device)

    def __call__(self, logits: torch.Tensor, temperatures: torch.Tensor | None, all_greedy: bool,
                 out: torch.Tensor | None = None) -> torch.Tensor:
        if all_greedy:
            self.seed.add_(1)
            return greedy_argmax(logits, out=out)
        return sample(logits, temperatures, self.seed, out=out)
