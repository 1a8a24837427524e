"""Token sampler (kavor/layers/sampler.py:7-66).

Greedy rows (temperature 0) take the argmax of the logits, first index on ties, as
torch.argmax and the reference kernel do; an all-greedy batch is one pass of the HIP
argmax kernel (kvp_argmax_bf16).  Other rows draw with the Gumbel-max trick,
argmax(logits / T + G) with G = -log(-log(U)), which samples softmax(logits / T)
exactly; the random stream (torch's Philox generator) differs from the reference's, so
sampled tokens at T > 0 are equal in distribution, not token for token.
"""

from __future__ import annotations

import torch

from kavor_amd.layers.fused import greedy_argmax


class Sampler:

    def __call__(self, logits: torch.Tensor, temperatures: torch.Tensor, all_greedy: bool) -> torch.Tensor:
        if all_greedy:
            return greedy_argmax(logits)
        scores = logits.float()
        t = temperatures.to(scores.device, torch.float32).unsqueeze(1)
        u = torch.rand_like(scores).clamp_(min=1e-30, max=1.0 - 1e-7)
        gumbel = -torch.log(-torch.log(u))
        sampled = torch.where(t > 0, scores / t.clamp_min(1e-30) + gumbel, scores)
        return sampled.argmax(dim=-1)
