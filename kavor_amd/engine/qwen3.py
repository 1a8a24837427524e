"""Qwen3 decoder that drives the paged KV path end to end.

The model is the caller of the path (kavor/models/qwen3.py:75-91).  Per layer:

  add-RMSNorm (HIP) -> qkv GEMM -> fused q/k RMSNorm + RoPE + K/V append (HIP)
  -> paged attention over the page pool (HIP) -> o GEMM -> add-RMSNorm (HIP)
  -> gate_up GEMM -> SiLU * up (HIP) -> down GEMM

In decode the q/k norm + RoPE + append and the paged attention are one launch
(kvp_paged_decode_fused_bf16) unless fused_decode is off.

With caller="dropin" the attention block keeps the reference's order instead: q/k
RMSNorm + RoPE (HIP, k into a fresh tensor), then Attention.forward(q, k, v) with v a
view of the qkv rows, which appends k / v (store_kvcache) and runs varlen prefill
(dense, or paged when the batch has cached prefixes) or paged decode.

GEMMs are torch (hipBLASLt); every other op is a kernel of libkvpath.so
(kavor_amd.layers.fused, kavor_amd.layers.attention), with the reference's numerics:
RMSNorm statistics in fp32 and the normalised value rounded to bf16 before the weight
(kavor/layers/layernorm.py:235-284), neox RoPE in fp32 (rotary_embedding.py:8-53), SiLU in
fp32 (activation.py:6-11).  Because k and v go straight from the qkv rows into the
pages, prefill attention always reads the pages in the fused order (the runner always
passes block tables), which is the reference's prefix-cache mode
(flash_attention_kvcache.py:74-79) applied to every prefill.  The embedding / LM head are tied; during prefill only each
sequence's last token is projected to logits (kavor/layers/embed_head.py:56-66).
"""

from __future__ import annotations

import json
import math
from dataclasses import asdict, dataclass, fields
from pathlib import Path

import torch
import torch.nn.functional as F
from torch import nn

from kavor_amd.layers import fused
from kavor_amd.layers.attention import Attention, paged_decode_fused
from kavor_amd.utils.context import get_context


@dataclass
class Qwen3Spec:
    """Architecture hyper-parameters (the Hugging Face Qwen3 config.json fields used)."""

    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    max_position_embeddings: int = 40960
    tie_word_embeddings: bool = True
    attention_bias: bool = False
    hidden_act: str = "silu"
    eos_token_id: int = 151645

    @classmethod
    def qwen3_0_6b(cls) -> "Qwen3Spec":
        return cls()

    @classmethod
    def from_dict(cls, cfg: dict) -> "Qwen3Spec":
        names = {f.name for f in fields(cls)}
        values = {k: v for k, v in cfg.items() if k in names}
        if isinstance(values.get("eos_token_id"), list):
            values["eos_token_id"] = values["eos_token_id"][0]
        rope_scaling = cfg.get("rope_scaling")
        if isinstance(rope_scaling, dict) and "rope_theta" in rope_scaling:
            values["rope_theta"] = rope_scaling["rope_theta"]
        if values.get("attention_bias", False):
            raise ValueError("Qwen3 with qkv bias is not supported (Qwen3 checkpoints use q/k norm)")
        if values.get("hidden_act", "silu") != "silu":
            raise ValueError(f"unsupported activation {values['hidden_act']}")
        return cls(**values)

    @classmethod
    def from_pretrained(cls, path: str | Path) -> "Qwen3Spec":
        with open(Path(path) / "config.json") as f:
            return cls.from_dict(json.load(f))

    def to_hf_dict(self) -> dict:
        d = asdict(self)
        d.update(architectures=["Qwen3ForCausalLM"], model_type="qwen3", torch_dtype="bfloat16")
        return d


# ------------------------------------------------------------------ layers

def rope_cache(head_dim: int, max_position: int, base: float, device) -> torch.Tensor:
    """[max_position, head_dim] fp32: cos of each frequency in the first half, sin in the
    second (the cos_sin_cache of rotary_embedding.py:56-66, without its head axis)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    t = torch.arange(max_position, dtype=torch.float32, device=device)
    freqs = torch.outer(t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).contiguous()


class RMSNorm(nn.Module):

    def __init__(self, size: int, eps: float, device=None, dtype=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(size, device=device, dtype=dtype), requires_grad=False)

    def forward(self, x, residual=None):
        if residual is None:
            return fused.rms_norm(x, self.weight, self.eps)
        return fused.add_rms_norm(x, residual, self.weight, self.eps)


def _weight(*shape, device, dtype) -> nn.Parameter:
    return nn.Parameter(torch.empty(*shape, device=device, dtype=dtype), requires_grad=False)


class Qwen3Attention(nn.Module):

    def __init__(self, spec: Qwen3Spec, rope: torch.Tensor, device, dtype, caller: str = "fused",
                 fused_decode: bool = True):
        super().__init__()
        self.caller = caller
        self.fused_decode = fused_decode and caller == "fused"
        self.num_heads = spec.num_attention_heads
        self.num_kv_heads = spec.num_key_value_heads
        self.head_dim = spec.head_dim
        self.q_size = self.num_heads * self.head_dim
        self.kv_size = self.num_kv_heads * self.head_dim
        self.qkv_proj = _weight(self.q_size + 2 * self.kv_size, spec.hidden_size, device=device, dtype=dtype)
        self.o_proj = _weight(spec.hidden_size, self.q_size, device=device, dtype=dtype)
        self.q_norm = RMSNorm(self.head_dim, spec.rms_norm_eps, device, dtype)
        self.k_norm = RMSNorm(self.head_dim, spec.rms_norm_eps, device, dtype)
        self.rope = rope
        self.attn = Attention(self.num_heads, self.head_dim, self.head_dim ** -0.5, self.num_kv_heads)

    def forward(self, positions: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
        qkv = F.linear(hidden, self.qkv_proj)
        if self.caller == "dropin":
            return self.forward_dropin(positions, qkv)
        attn = self.attn
        k_cache, v_cache = attn.k_cache[0], attn.v_cache[0]
        bound = k_cache.numel() > 0 and v_cache.numel() > 0
        context = get_context()
        if self.fused_decode and bound and not context.is_prefill:
            # q/k norm + RoPE + append + paged decode in one launch
            o = paged_decode_fused(qkv, self.rope, self.q_norm.weight, self.k_norm.weight,
                                   self.q_norm.eps, self.num_heads, self.num_kv_heads, k_cache, v_cache,
                                   context.slot_mapping, context.context_lens, context.block_tables,
                                   attn.scale)
            return F.linear(o.reshape(qkv.shape[0], self.q_size), self.o_proj)
        q = fused.qk_norm_rope_append(
            qkv, positions, self.rope, self.q_norm.weight, self.k_norm.weight, self.q_norm.eps,
            self.num_heads, self.num_kv_heads, k_cache if bound else None, v_cache if bound else None,
            get_context().slot_mapping if bound else None)
        o = attn.forward_cached(q)
        return F.linear(o.reshape(q.shape[0], self.q_size), self.o_proj)

    def forward_dropin(self, positions: torch.Tensor, qkv: torch.Tensor) -> torch.Tensor:
        """The reference's caller order (kavor/models/qwen3.py:80-90): q_norm, k_norm and
        rotary_emb (one HIP launch; k comes out contiguous with row stride Hkv*D), v a
        strided view of the qkv rows (row stride (Hq+2Hkv)*D), then attn(q, k, v)."""
        T = qkv.shape[0]
        q, k = fused.qk_norm_rope(qkv, positions, self.rope, self.q_norm.weight, self.k_norm.weight,
                                  self.q_norm.eps, self.num_heads, self.num_kv_heads)
        v = qkv[:, self.q_size + self.kv_size:].view(T, self.num_kv_heads, self.head_dim)
        o = self.attn(q, k, v)
        return F.linear(o.reshape(T, self.q_size), self.o_proj)


class Qwen3MLP(nn.Module):

    def __init__(self, spec: Qwen3Spec, device, dtype):
        super().__init__()
        self.intermediate_size = spec.intermediate_size
        self.gate_up_proj = _weight(2 * spec.intermediate_size, spec.hidden_size, device=device, dtype=dtype)
        self.down_proj = _weight(spec.hidden_size, spec.intermediate_size, device=device, dtype=dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.linear(fused.silu_and_mul(F.linear(x, self.gate_up_proj)), self.down_proj)


class Qwen3DecoderLayer(nn.Module):

    def __init__(self, spec: Qwen3Spec, rope: torch.Tensor, device, dtype, caller: str = "fused",
                 fused_decode: bool = True):
        super().__init__()
        self.self_attn = Qwen3Attention(spec, rope, device, dtype, caller, fused_decode)
        self.mlp = Qwen3MLP(spec, device, dtype)
        self.input_layernorm = RMSNorm(spec.hidden_size, spec.rms_norm_eps, device, dtype)
        self.post_attention_layernorm = RMSNorm(spec.hidden_size, spec.rms_norm_eps, device, dtype)

    def forward(self, positions, hidden, residual):
        if residual is None:
            hidden, residual = self.input_layernorm(hidden), hidden
        else:
            hidden, residual = self.input_layernorm(hidden, residual)
        hidden = self.self_attn(positions, hidden)
        hidden, residual = self.post_attention_layernorm(hidden, residual)
        return self.mlp(hidden), residual


class Qwen3ForCausalLM(nn.Module):
    """Qwen3 causal LM over the paged KV cache (bf16 weights on one GPU)."""

    def __init__(self, spec: Qwen3Spec, device, dtype=torch.bfloat16, caller: str = "fused",
                 fused_decode: bool = True):
        super().__init__()
        self.spec = spec
        # prefill attention reads the pages (block tables on every prefill) when the layers
        # append k / v before attention; the drop-in order attends over fresh k / v unless
        # a prefix is cached
        self.prefill_reads_pages = caller == "fused"
        rope = rope_cache(spec.head_dim, spec.max_position_embeddings, spec.rope_theta, device)
        self.register_buffer("rope_table", rope, persistent=False)
        self.embed_tokens = _weight(spec.vocab_size, spec.hidden_size, device=device, dtype=dtype)
        self.layers = nn.ModuleList(
            [Qwen3DecoderLayer(spec, rope, device, dtype, caller, fused_decode)
             for _ in range(spec.num_hidden_layers)])
        self.norm = RMSNorm(spec.hidden_size, spec.rms_norm_eps, device, dtype)
        self.lm_head = (self.embed_tokens if spec.tie_word_embeddings
                        else _weight(spec.vocab_size, spec.hidden_size, device=device, dtype=dtype))

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        hidden = F.embedding(input_ids, self.embed_tokens)
        residual = None
        for layer in self.layers:
            hidden, residual = layer(positions, hidden, residual)
        hidden, _ = self.norm(hidden, residual)
        return hidden

    def compute_logits(self, hidden: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        context = get_context()
        if context.is_prefill:
            hidden = hidden[context.cu_seqlens_q[1:] - 1]
        if out is not None:
            return torch.mm(hidden, self.lm_head.t(), out=out)
        return F.linear(hidden, self.lm_head)

    # ------------------------------------------------------------------ weights

    def named_weights(self) -> dict[str, torch.Tensor]:
        """Parameters under this module's own names (the fused qkv / gate_up layout)."""
        return {n: p for n, p in self.named_parameters()}

    @torch.no_grad()
    def init_random(self, seed: int = 0, std: float = 0.02) -> None:
        """Deterministic random weights: N(0, std) matrices, unit norm weights."""
        gen = torch.Generator(device=self.embed_tokens.device).manual_seed(seed)
        for name, p in self.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.normal_(0.0, std, generator=gen)

    @torch.no_grad()
    def load_hf_state(self, tensors: dict[str, torch.Tensor]) -> None:
        """Loads Hugging Face Qwen3 tensor names, fusing q/k/v and gate/up; every
        parameter must be present (a missing one raises, like the reference loader)."""
        spec = self.spec
        used = set()

        def take(name):
            if name not in tensors:
                raise KeyError(f"checkpoint is missing {name}")
            used.add(name)
            return tensors[name]

        self.embed_tokens.copy_(take("model.embed_tokens.weight"))
        self.norm.weight.copy_(take("model.norm.weight"))
        if not spec.tie_word_embeddings:
            self.lm_head.copy_(take("lm_head.weight"))
        for i, layer in enumerate(self.layers):
            pre = f"model.layers.{i}."
            a = layer.self_attn
            q, kv = a.q_size, a.kv_size
            a.qkv_proj[:q].copy_(take(pre + "self_attn.q_proj.weight"))
            a.qkv_proj[q:q + kv].copy_(take(pre + "self_attn.k_proj.weight"))
            a.qkv_proj[q + kv:].copy_(take(pre + "self_attn.v_proj.weight"))
            a.o_proj.copy_(take(pre + "self_attn.o_proj.weight"))
            a.q_norm.weight.copy_(take(pre + "self_attn.q_norm.weight"))
            a.k_norm.weight.copy_(take(pre + "self_attn.k_norm.weight"))
            m = layer.mlp
            I = m.intermediate_size
            m.gate_up_proj[:I].copy_(take(pre + "mlp.gate_proj.weight"))
            m.gate_up_proj[I:].copy_(take(pre + "mlp.up_proj.weight"))
            m.down_proj.copy_(take(pre + "mlp.down_proj.weight"))
            layer.input_layernorm.weight.copy_(take(pre + "input_layernorm.weight"))
            layer.post_attention_layernorm.weight.copy_(take(pre + "post_attention_layernorm.weight"))
        extra = set(tensors) - used - {"lm_head.weight"}
        if extra:
            raise KeyError(f"checkpoint has tensors this model does not use: {sorted(extra)[:5]}")


def hf_tensor_shapes(spec: Qwen3Spec) -> dict[str, tuple[int, ...]]:
    """Hugging Face tensor names and shapes of a Qwen3 checkpoint with this spec."""
    H, D = spec.hidden_size, spec.head_dim
    q, kv, I = spec.num_attention_heads * D, spec.num_key_value_heads * D, spec.intermediate_size
    shapes = {"model.embed_tokens.weight": (spec.vocab_size, H), "model.norm.weight": (H,)}
    if not spec.tie_word_embeddings:
        shapes["lm_head.weight"] = (spec.vocab_size, H)
    for i in range(spec.num_hidden_layers):
        pre = f"model.layers.{i}."
        shapes.update({
            pre + "self_attn.q_proj.weight": (q, H),
            pre + "self_attn.k_proj.weight": (kv, H),
            pre + "self_attn.v_proj.weight": (kv, H),
            pre + "self_attn.o_proj.weight": (H, q),
            pre + "self_attn.q_norm.weight": (D,),
            pre + "self_attn.k_norm.weight": (D,),
            pre + "mlp.gate_proj.weight": (I, H),
            pre + "mlp.up_proj.weight": (I, H),
            pre + "mlp.down_proj.weight": (H, I),
            pre + "input_layernorm.weight": (H,),
            pre + "post_attention_layernorm.weight": (H,),
        })
    return shapes


def write_random_checkpoint(path: str | Path, spec: Qwen3Spec, seed: int = 0, std: float = 0.02) -> Path:
    """Writes config.json + model.safetensors with random bf16 weights (CPU, seeded)."""
    from safetensors.torch import save_file

    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    gen = torch.Generator().manual_seed(seed)
    tensors = {}
    for name, shape in hf_tensor_shapes(spec).items():
        if name.endswith("norm.weight"):
            t = torch.ones(shape, dtype=torch.bfloat16)
        else:
            t = (torch.randn(shape, generator=gen) * std).to(torch.bfloat16)
        tensors[name] = t
    save_file(tensors, str(path / "model.safetensors"), metadata={"format": "pt"})
    with open(path / "config.json", "w") as f:
        json.dump(spec.to_hf_dict(), f, indent=1)
    return path


def load_checkpoint_tensors(path: str | Path) -> dict[str, torch.Tensor]:
    """Reads every *.safetensors file of a checkpoint directory (no pickle)."""
    from safetensors.torch import load_file

    files = sorted(Path(path).glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no *.safetensors in {path}")
    tensors = {}
    for f in files:
        tensors.update(load_file(str(f)))
    return tensors


def num_parameters(spec: Qwen3Spec) -> int:
    return sum(math.prod(s) for s in hf_tensor_shapes(spec).values())
