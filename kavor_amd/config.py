"""Engine configuration (kavor/config.py:17-58, single-GPU text models).

Same field names and defaults as the reference.  `model` is either a checkpoint
directory (Hugging Face config.json + *.safetensors) or a Qwen3Spec, in which case the
weights are random (seeded by `seed`).  Differences from the reference:

- tensor_parallel_size must be 1: this engine drives one GPU;
- kvcache_block_size must be a multiple of 64 (the page size the HIP kernels tile by;
  the reference requires multiples of 256 because flash-attn does, config.py:42);
- num_kvcache_blocks > 0 fixes the page-pool size instead of sizing it from
  gpu_memory_utilization;
- attention_caller picks how the Qwen3 layers call the paged path: "fused" (one kernel
  normalises, rotates and appends k / v, then attention reads the pages) or "dropin"
  (the reference's order, kavor/models/qwen3.py:85-90: q/k norm + RoPE, then
  Attention.forward(q, k, v) appends through store_kvcache and runs dense varlen
  prefill for batches without a cached prefix);
- fused_decode (with the fused caller) runs a decode step's q/k norm + RoPE, K/V append
  and paged attention as one launch per layer instead of two.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field

from kavor_amd.engine.qwen3 import Qwen3Spec


@dataclass
class Config:
    model: str | Qwen3Spec | None = None
    max_num_batched_tokens: int = 16384
    max_num_seqs: int = 512
    max_model_len: int = 4096
    gpu_memory_utilization: float = 0.9
    tensor_parallel_size: int = 1
    enforce_eager: bool = False
    profile: bool = False
    eos: int = -1
    kvcache_block_size: int = 256
    num_kvcache_blocks: int = -1
    seed: int = 0
    attention_caller: str = "fused"
    fused_decode: bool = True
    spec: Qwen3Spec = field(init=False)
    checkpoint: str | None = field(init=False, default=None)

    def __post_init__(self):
        if isinstance(self.model, Qwen3Spec):
            self.spec = self.model
        elif self.model is None:
            self.spec = Qwen3Spec.qwen3_0_6b()
        else:
            if not os.path.isdir(self.model):
                raise RuntimeError(f"Model not found: {self.model}")
            self.spec = Qwen3Spec.from_pretrained(self.model)
            self.checkpoint = str(self.model)
        if self.tensor_parallel_size != 1:
            raise ValueError("this engine runs on one GPU: tensor_parallel_size must be 1")
        if self.kvcache_block_size % 64 != 0 or self.kvcache_block_size <= 0:
            raise ValueError(f"kvcache_block_size must be a positive multiple of 64, "
                             f"got {self.kvcache_block_size}")
        if self.attention_caller not in ("fused", "dropin"):
            raise ValueError(f"attention_caller must be 'fused' or 'dropin', got {self.attention_caller!r}")
        if not 0.0 < self.gpu_memory_utilization <= 1.0:
            raise ValueError("gpu_memory_utilization must be in (0, 1]")
        if self.max_num_seqs < 1 or self.max_num_batched_tokens < 1:
            raise ValueError("max_num_seqs and max_num_batched_tokens must be positive")
        self.max_model_len = min(self.max_model_len, self.spec.max_position_embeddings)
        if self.eos == -1:
            self.eos = self.spec.eos_token_id
