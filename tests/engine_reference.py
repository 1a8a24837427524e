"""Full-sequence fp32-attention forward of a Qwen3ForCausalLM, for checking the engine.

Recomputes the logits of every position of a token sequence with the model's own
weights, the oracle's restatements of the reference layers (oracle/layers_oracle.py)
and attention as a causal fp32 scaled-dot-product over the whole sequence: no kernel of
libkvpath.so is involved, only torch GEMMs.  A token the
engine generated greedily is accepted when its reference logit is within `tol` of the
reference maximum at that position (near-ties may legitimately flip under bf16).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle.layers_oracle import add_rms_norm, apply_rope, rms_norm, silu_and_mul


@torch.inference_mode()
def reference_logits(model, token_ids: list[int]) -> torch.Tensor:
    spec = model.spec
    dev = model.embed_tokens.device
    ids = torch.tensor(token_ids, dtype=torch.int64, device=dev)
    T = ids.numel()
    pos = torch.arange(T, device=dev)
    cos, sin = model.rope_table[pos].unsqueeze(1).chunk(2, dim=-1)
    G = spec.num_attention_heads // spec.num_key_value_heads
    h = F.embedding(ids, model.embed_tokens)
    residual = None
    for layer in model.layers:
        if residual is None:
            x, residual = rms_norm(h, layer.input_layernorm.weight, spec.rms_norm_eps), h
        else:
            x, residual = add_rms_norm(h, residual, layer.input_layernorm.weight, spec.rms_norm_eps)
        a = layer.self_attn
        q, k, v = F.linear(x, a.qkv_proj).split([a.q_size, a.kv_size, a.kv_size], dim=-1)
        q = rms_norm(q.view(T, -1, spec.head_dim), a.q_norm.weight, spec.rms_norm_eps)
        k = rms_norm(k.view(T, -1, spec.head_dim), a.k_norm.weight, spec.rms_norm_eps)
        v = v.view(T, -1, spec.head_dim)
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        qf = q.float().transpose(0, 1)
        kf = k.float().repeat_interleave(G, dim=1).transpose(0, 1)
        vf = v.float().repeat_interleave(G, dim=1).transpose(0, 1)
        o = F.scaled_dot_product_attention(qf, kf, vf, is_causal=True, scale=spec.head_dim ** -0.5)
        o = o.transpose(0, 1).to(torch.bfloat16).reshape(T, -1)
        h = F.linear(o, a.o_proj)
        x, residual = add_rms_norm(h, residual, layer.post_attention_layernorm.weight, spec.rms_norm_eps)
        h = F.linear(silu_and_mul(F.linear(x, layer.mlp.gate_up_proj)), layer.mlp.down_proj)
    h, _ = add_rms_norm(h, residual, model.norm.weight, spec.rms_norm_eps)
    return F.linear(h, model.lm_head).float()


def check_greedy_tokens(model, prompt: list[int], completion: list[int], tol: float) -> float:
    """Asserts each greedy completion token is a reference argmax up to `tol`; returns
    the largest shortfall seen."""
    full = list(prompt) + list(completion)
    logits = reference_logits(model, full[:-1])
    worst = 0.0
    for j, tok in enumerate(completion):
        row = logits[len(prompt) - 1 + j]
        gap = float(row.max() - row[tok])
        worst = max(worst, gap)
        assert gap <= tol, (f"token {j} of the completion ({tok}) is {gap:.4f} below the "
                            f"reference maximum (argmax {int(row.argmax())})")
    return worst
