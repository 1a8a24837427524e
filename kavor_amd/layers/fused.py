"""Python boundary of the fused layer kernels in libkvpath.so (include/kvpath.h).

These replace the engine-side Triton kernels around the paged KV path:
  rms_norm / add_rms_norm   kavor/layers/layernorm.py:235-284 (RMSNorm.forward)
  qk_norm_rope_append       q_norm + k_norm + rotary_emb + store_kvcache of qwen3.py:85-89
  qk_norm_rope              q_norm + k_norm + rotary_emb of qwen3.py:85-88 (no append)
  silu_and_mul              kavor/layers/activation.py:6-11
  greedy_argmax             the temperature-0 path of kavor/layers/sampler.py:7-66
Each function only validates layouts and forwards pointers and strides to the C ABI on
the current stream; there is no host computation and no fallback.
"""

from __future__ import annotations

import torch

from kavor_amd._lib import check, lib

__all__ = ["rms_norm", "add_rms_norm", "qk_norm_rope_append", "qk_norm_rope", "silu_and_mul",
           "greedy_argmax"]


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_bf16(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda or t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be a bf16 GPU tensor (got {t.dtype} on {t.device})")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must have a contiguous last dimension")


def _rows(t: torch.Tensor):
    """(num_tokens, rows_per_token, stride0, stride1) of a 2-D or 3-D view."""
    if t.dim() == 2:
        return t.shape[0], 1, t.stride(0), 0
    if t.dim() == 3:
        return t.shape[0], t.shape[1], t.stride(0), t.stride(1)
    raise ValueError(f"expected a 2-D or 3-D tensor, got shape {tuple(t.shape)}")


def _norm(x, weight, eps, residual, out):
    _check_bf16("x", x)
    _check_bf16("weight", weight)
    if weight.dim() != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError("weight must be 1-D with x.shape[-1] elements")
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _check_bf16("out", out)
    if out.shape != x.shape:
        raise ValueError("out must have x's shape")
    T, H, xs0, xs1 = _rows(x)
    _, _, os0, os1 = _rows(out)
    if residual is not None:
        _check_bf16("residual", residual)
        if residual.shape != x.shape:
            raise ValueError("residual must have x's shape")
        _, _, rs0, rs1 = _rows(residual)
        rptr = residual.data_ptr()
    else:
        rptr, rs0, rs1 = 0, 0, 0
    rc = lib().kvp_rmsnorm_bf16(x.data_ptr(), xs0, xs1, rptr, rs0, rs1, weight.data_ptr(), float(eps),
                                out.data_ptr(), os0, os1, T, H, x.shape[-1], _stream(x))
    check("kvp_rmsnorm_bf16", rc)
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm of the last dimension of a 2-D or 3-D bf16 view (strided rows allowed)."""
    return _norm(x, weight, eps, None, out)


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float,
                 out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """residual <- bf16(x + residual) in place; returns (RMSNorm of the fp32 sum, residual)."""
    return _norm(x, weight, eps, residual, out), residual


def qk_norm_rope_append(qkv: torch.Tensor, positions: torch.Tensor, cos_sin: torch.Tensor,
                        q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, eps: float,
                        num_q_heads: int, num_kv_heads: int,
                        k_cache: torch.Tensor | None, v_cache: torch.Tensor | None,
                        slot_mapping: torch.Tensor | None,
                        q_out: torch.Tensor | None = None) -> torch.Tensor:
    """q/k RMSNorm + neox RoPE of the fused qkv rows; returns q [T, Hq, 128] and appends
    the rotated k and the raw v to the paged caches at slot_mapping (skipped if None)."""
    _check_bf16("qkv", qkv)
    if qkv.dim() != 2:
        raise ValueError("qkv must be [num_tokens, (Hq + 2 Hkv) * head_dim]")
    T = qkv.shape[0]
    D = cos_sin.shape[1]
    if qkv.shape[1] != (num_q_heads + 2 * num_kv_heads) * D:
        raise ValueError("qkv width does not match the head counts and the RoPE table")
    if cos_sin.dtype != torch.float32 or not cos_sin.is_contiguous() or cos_sin.dim() != 2:
        raise ValueError("cos_sin must be a contiguous fp32 [max_position, head_dim] table")
    if positions.dtype != torch.int32 or not positions.is_contiguous() or positions.numel() != T:
        raise ValueError("positions must be a contiguous int32 tensor with one entry per token")
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        _check_bf16(name, w)
        if w.shape != (D,):
            raise ValueError(f"{name} must have head_dim elements")
    if q_out is None:
        q_out = torch.empty(T, num_q_heads, D, dtype=torch.bfloat16, device=qkv.device)
    _check_bf16("q_out", q_out)
    if q_out.shape != (T, num_q_heads, D) or q_out.stride(1) != D:
        raise ValueError("q_out must be [T, Hq, head_dim] with contiguous heads")
    if slot_mapping is not None:
        if slot_mapping.dtype != torch.int32 or not slot_mapping.is_contiguous() or slot_mapping.numel() != T:
            raise ValueError("slot_mapping must be a contiguous int32 tensor with one entry per token")
        _check_bf16("k_cache", k_cache)
        _check_bf16("v_cache", v_cache)
        if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
            raise ValueError("k_cache and v_cache must share shape and strides")
        if k_cache.shape[2:] != (num_kv_heads, D):
            raise ValueError("cache heads / head_dim do not match")
        nb, bs = k_cache.shape[0], k_cache.shape[1]
        cache = (k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
                 k_cache.stride(2), nb * bs)
        sm, block_size = slot_mapping.data_ptr(), bs
    else:
        cache, sm, block_size = (0, 0, 0, 0, 0, 0), 0, 1
    rc = lib().kvp_qk_norm_rope_append_bf16(
        qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), cos_sin.data_ptr(), cos_sin.shape[0],
        q_norm_weight.data_ptr(), k_norm_weight.data_ptr(), float(eps),
        q_out.data_ptr(), q_out.stride(0), *cache, sm, T, num_q_heads, num_kv_heads, D,
        block_size, _stream(qkv))
    check("kvp_qk_norm_rope_append_bf16", rc)
    return q_out


def qk_norm_rope(qkv: torch.Tensor, positions: torch.Tensor, cos_sin: torch.Tensor,
                 q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, eps: float,
                 num_q_heads: int, num_kv_heads: int) -> tuple[torch.Tensor, torch.Tensor]:
    """q/k RMSNorm + neox RoPE of the fused qkv rows without the append: returns fresh
    q [T, Hq, 128] and k [T, Hkv, 128] (the q_norm, k_norm and rotary_emb of
    kavor/models/qwen3.py:85-88, one launch); v stays a view of qkv."""
    _check_bf16("qkv", qkv)
    if qkv.dim() != 2:
        raise ValueError("qkv must be [num_tokens, (Hq + 2 Hkv) * head_dim]")
    T = qkv.shape[0]
    D = cos_sin.shape[1]
    if qkv.shape[1] < (num_q_heads + num_kv_heads) * D:
        raise ValueError("qkv is narrower than the q and k heads")
    if cos_sin.dtype != torch.float32 or not cos_sin.is_contiguous() or cos_sin.dim() != 2:
        raise ValueError("cos_sin must be a contiguous fp32 [max_position, head_dim] table")
    if positions.dtype != torch.int32 or not positions.is_contiguous() or positions.numel() != T:
        raise ValueError("positions must be a contiguous int32 tensor with one entry per token")
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        _check_bf16(name, w)
        if w.shape != (D,):
            raise ValueError(f"{name} must have head_dim elements")
    q = torch.empty(T, num_q_heads, D, dtype=torch.bfloat16, device=qkv.device)
    k = torch.empty(T, num_kv_heads, D, dtype=torch.bfloat16, device=qkv.device)
    rc = lib().kvp_qk_norm_rope_bf16(
        qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), cos_sin.data_ptr(), cos_sin.shape[0],
        q_norm_weight.data_ptr(), k_norm_weight.data_ptr(), float(eps),
        q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), T, num_q_heads, num_kv_heads, D,
        _stream(qkv))
    check("kvp_qk_norm_rope_bf16", rc)
    return q, k


def silu_and_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """SiLU(gate) * up for gate_up = [gate | up] along the last dimension."""
    _check_bf16("gate_up", gate_up)
    if gate_up.dim() != 2 or gate_up.shape[1] % 2:
        raise ValueError("gate_up must be [num_tokens, 2 * intermediate]")
    T, I = gate_up.shape[0], gate_up.shape[1] // 2
    if out is None:
        out = torch.empty(T, I, dtype=torch.bfloat16, device=gate_up.device)
    _check_bf16("out", out)
    if out.shape != (T, I):
        raise ValueError("out must be [num_tokens, intermediate]")
    rc = lib().kvp_silu_mul_bf16(gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(), out.stride(0),
                                 T, I, _stream(gate_up))
    check("kvp_silu_mul_bf16", rc)
    return out


_argmax_workspaces: dict[int, torch.Tensor] = {}
# The largest split-row workspace any batch needs (fewer than 192 rows, up to 16 segments
# of one 8-byte key each, at most 1024 keys); reserved once per device.
_ARGMAX_WORKSPACE_BYTES = 16384


def argmax_workspace(device: torch.device) -> torch.Tensor:
    """The per-device workspace of the split-row argmax, allocated on first use (which the
    engine makes before any graph capture)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    ws = _argmax_workspaces.get(index)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("the argmax workspace must be reserved before graph capture: "
                               "call argmax_workspace(device) first")
        ws = torch.empty(_ARGMAX_WORKSPACE_BYTES, dtype=torch.uint8, device=torch.device("cuda", index))
        _argmax_workspaces[index] = ws
    return ws


def greedy_argmax(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """int64 index of each row's maximum (first on ties, NaN largest)."""
    _check_bf16("logits", logits)
    if logits.dim() != 2:
        raise ValueError("logits must be [num_rows, vocab]")
    if out is None:
        out = torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
    if out.dtype != torch.int64 or not out.is_contiguous() or out.numel() != logits.shape[0]:
        raise ValueError("out must be a contiguous int64 tensor with one entry per row")
    ws = argmax_workspace(logits.device)
    need = lib().kvp_argmax_workspace_bytes(logits.shape[0])
    if need > ws.numel():
        raise RuntimeError(f"argmax workspace of {ws.numel()} bytes, {need} needed")
    rc = lib().kvp_argmax_bf16(logits.data_ptr(), logits.stride(0), logits.shape[0], logits.shape[1],
                               out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(logits))
    check("kvp_argmax_bf16", rc)
    return out


def sample(logits: torch.Tensor, temperatures: torch.Tensor, seed: torch.Tensor,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """int64 token per row: a Gumbel-max sample of softmax(logits / T) for rows with
    T > 0, the greedy index for the others (kavor/layers/sampler.py:7-66).  seed is a
    device int32 scalar that the call advances by one before drawing, as the reference's
    Sampler.forward does, so that a captured graph draws new noise on every replay."""
    _check_bf16("logits", logits)
    if logits.dim() != 2:
        raise ValueError("logits must be [num_rows, vocab]")
    n = logits.shape[0]
    if temperatures.dtype != torch.float32 or not temperatures.is_contiguous() or temperatures.numel() < n \
            or temperatures.device != logits.device:
        raise ValueError("temperatures must be a contiguous fp32 tensor on the logits' device, one per row")
    if seed.dtype != torch.int32 or seed.numel() != 1 or seed.device != logits.device:
        raise ValueError("seed must be a one-element int32 tensor on the logits' device")
    if out is None:
        out = torch.empty(n, dtype=torch.int64, device=logits.device)
    if out.dtype != torch.int64 or not out.is_contiguous() or out.numel() != n:
        raise ValueError("out must be a contiguous int64 tensor with one entry per row")
    ws = argmax_workspace(logits.device)
    need = lib().kvp_argmax_workspace_bytes(n)
    if need > ws.numel():
        raise RuntimeError(f"argmax workspace of {ws.numel()} bytes, {need} needed")
    seed.add_(1)
    rc = lib().kvp_sample_bf16(logits.data_ptr(), logits.stride(0), n, logits.shape[1], temperatures.data_ptr(),
                               seed.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(logits))
    check("kvp_sample_bf16", rc)
    return out
