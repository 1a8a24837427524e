"""Per-request sampling parameters (kavor/sampling_params.py:5-13).

Same fields and defaults as the reference.  One deliberate difference: temperature 0
is accepted and means greedy decoding (argmax, first index on ties).  The reference
rejects temperatures <= 1e-10 in SamplingParams (sampling_params.py:11) although its
sampler kernel already treats 0 as greedy (kavor/layers/sampler.py:34-38); the
end-to-end Qwen3-0.6B workload is specified greedy, so the engine here allows it.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(slots=True)
class SamplingParams:
    temperature: float = 1.0
    max_tokens: int = 64
    ignore_eos: bool = False

    def __post_init__(self):
        if not self.temperature >= 0.0:
            raise ValueError(f"temperature must be >= 0 (0 = greedy), got {self.temperature}")
        if self.max_tokens < 1:
            raise ValueError(f"max_tokens must be >= 1, got {self.max_tokens}")
