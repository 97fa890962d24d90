"""Trusted forwards, restated from the reference (test infrastructure only).

Each function is the mathematics the reference's oracle differentiates; the
citation names the file it restates.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def softmax_forward_ref(x: torch.Tensor) -> torch.Tensor:
    """src/evograd/ops/level1/softmax/forward_ref.py:6-7."""
    return torch.softmax(x.float(), dim=-1).to(x.dtype)


def rmsnorm_forward_ref(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """src/evograd/ops/level1/rmsnorm/forward_ref.py:6-21."""
    if x.ndim != 2:
        raise ValueError(f"expected x to be 2D, got shape {tuple(x.shape)}")
    if weight.ndim != 1 or weight.shape[0] != x.shape[1]:
        raise ValueError("weight must be 1D with length hidden")
    x32 = x.float()
    ms = torch.mean(x32 * x32, dim=-1, keepdim=True)
    x_hat = x32 * torch.rsqrt(ms + eps)
    return (x_hat * weight.float()).to(x.dtype)


def rmsnorm_runtime_ref(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """src/evograd/ops/level1/rmsnorm/forward_ref.py:24-34 (the fused spelling timed
    as the eager baseline)."""
    return F.rms_norm(x, (x.shape[-1],), weight=weight, eps=eps)


def fused_add_rms_norm_forward_ref(x: torch.Tensor, residual: torch.Tensor,
                                   weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """src/evograd/ops/level2/fused_add_rms_norm/forward_ref.py:6-16: the sum in the
    input dtype, its mean square in fp32, then (s * rstd) * weight with rstd cast
    to the sum's dtype."""
    if x.shape != residual.shape or x.ndim != 2:
        raise ValueError("x and residual must be equal 2D tensors")
    summed = x + residual
    rstd = torch.rsqrt(summed.float().pow(2).mean(dim=-1, keepdim=True) + eps)
    return (summed * rstd.to(summed.dtype)) * weight


def fused_add_rms_norm_runtime_ref(x: torch.Tensor, residual: torch.Tensor,
                                   weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """src/evograd/ops/level2/fused_add_rms_norm/forward_ref.py:19-34: the add, then
    the fused F.rms_norm (the eager baseline's spelling)."""
    return F.rms_norm(x + residual, (x.shape[-1],), weight=weight, eps=eps)


def layernorm_forward_ref(x, weight, bias, eps: float = 1e-5):
    """src/evograd/ops/level1/layernorm/forward_ref.py:6-23."""
    if x.ndim != 2:
        raise ValueError(f"expected x to be 2D, got shape {tuple(x.shape)}")
    if weight.ndim != 1 or bias.ndim != 1:
        raise ValueError("weight and bias must be 1D tensors")
    x32 = x.float()
    mean = torch.mean(x32, dim=-1, keepdim=True)
    var = torch.mean((x32 - mean) ** 2, dim=-1, keepdim=True)
    x_hat = (x32 - mean) * torch.rsqrt(var + eps)
    return (x_hat * weight.float() + bias.float()).to(x.dtype)


def layernorm_runtime_ref(x, weight, bias, eps: float = 1e-5):
    """src/evograd/ops/level1/layernorm/forward_ref.py:26-42."""
    return F.layer_norm(x, (x.shape[-1],), weight=weight, bias=bias, eps=eps)


def swiglu_forward_ref(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """src/evograd/ops/level1/swiglu/forward_ref.py:6-9."""
    if a.shape != b.shape:
        raise ValueError(f"a and b must have the same shape, got {a.shape} and {b.shape}")
    return F.silu(a.float()).to(a.dtype) * b


def _rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def rope_forward_ref(x, cos, sin):
    """src/evograd/ops/level1/rope/forward_ref.py:28-47 (half-rotated layout)."""
    if x.ndim != 4:
        raise ValueError(f"rope expects [batch, heads, tokens, head_dim], got {tuple(x.shape)}")
    c = cos[None, None].float()
    s = sin[None, None].float()
    x32 = x.float()
    return (x32 * c + _rotate_half(x32) * s).to(x.dtype)


def causal_attention_forward_ref(q, k, v):
    """Causal SDPA written out: softmax(q k^T / sqrt(D) + mask) v, the semantics of
    F.scaled_dot_product_attention(q, k, v, is_causal=True) at
    src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:107. Scores and
    probabilities in fp32; the result is cast to q's dtype."""
    S, D = q.shape[-2], q.shape[-1]
    scale = 1.0 / (D ** 0.5)
    s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) * scale
    mask = torch.ones(S, S, dtype=torch.bool, device=q.device).triu_(1)
    s = s.masked_fill(mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v.float()).to(q.dtype)


def causal_attention_runtime_ref(q, k, v):
    """The eager PyTorch call the reference makes (llama3_decoder_layer/forward_ref.py:107)."""
    return F.scaled_dot_product_attention(q, k, v, is_causal=True)


def causal_attention_gqa_forward_ref(q, k, v):
    """src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:101-107: each kv
    head repeated over its group of query heads (repeat_interleave on the head
    axis), then causal attention."""
    repeat = q.shape[1] // k.shape[1]
    if repeat * k.shape[1] != q.shape[1]:
        raise ValueError("query heads must be a multiple of kv heads")
    if repeat > 1:
        k = k.repeat_interleave(repeat, dim=1)
        v = v.repeat_interleave(repeat, dim=1)
    return causal_attention_forward_ref(q, k, v)


def causal_attention_gqa_runtime_ref(q, k, v):
    """The reference's eager spelling: repeat_interleave, then F.sdpa (:101-107)."""
    repeat = q.shape[1] // k.shape[1]
    if repeat > 1:
        k = k.repeat_interleave(repeat, dim=1)
        v = v.repeat_interleave(repeat, dim=1)
    return F.scaled_dot_product_attention(q, k, v, is_causal=True)


def llama3_attention_forward_ref(q, k, v, cos, sin):
    """The attention half of src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:
    93-107: q and k rotated by _apply_rope (:42-51, the half-rotated RoPE in fp32 cast
    back to the input dtype, as rope_forward_ref), then each kv head repeated over its
    query group and causal attention."""
    return causal_attention_gqa_forward_ref(rope_forward_ref(q, cos, sin),
                                            rope_forward_ref(k, cos, sin), v)


def llama3_attention_runtime_ref(q, k, v, cos, sin):
    """The layer's eager spelling of the same half: _apply_rope, repeat_interleave and
    F.scaled_dot_product_attention(is_causal=True) (forward_ref.py:93-107)."""
    return causal_attention_gqa_runtime_ref(rope_forward_ref(q, cos, sin),
                                            rope_forward_ref(k, cos, sin), v)


def causal_attention_lse_ref(q, k):
    """logsumexp over keys of the scaled, causally masked scores, fp32 [B, H, S]:
    the statistic the attention forward saves."""
    S, D = q.shape[-2], q.shape[-1]
    s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) * (1.0 / D ** 0.5)
    mask = torch.ones(S, S, dtype=torch.bool, device=q.device).triu_(1)
    return torch.logsumexp(s.masked_fill(mask, float("-inf")), dim=-1)


def cross_entropy_forward_ref(logits: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """src/evograd/ops/level1/cross_entropy/forward_ref.py:6-12: mean hard-label cross
    entropy of the fp32-widened logits, ignore_index -100, cast to the logits dtype."""
    loss = F.cross_entropy(logits.float(), target, reduction="mean", ignore_index=-100)
    return loss.to(logits.dtype)


def fused_linear_cross_entropy_forward_ref(x: torch.Tensor, weight: torch.Tensor,
                                           target: torch.Tensor) -> torch.Tensor:
    """src/evograd/ops/level2/fused_linear_cross_entropy/forward_ref.py:23-35: fp32
    logits x @ weight.T, then the mean cross entropy (ignore_index -100 by default);
    the loss stays fp32."""
    logits = torch.matmul(x.float(), weight.float().t())
    return F.cross_entropy(logits, target, reduction="mean")


def _layer_rms_norm(x, weight, eps):
    """The decoder layer's RMSNorm (llama3_decoder_layer/forward_ref.py:36-40): fp32
    statistics, x * rrms cast back to x's dtype, then the gain in that dtype."""
    x32 = x.float()
    rrms = torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)
    return ((x32 * rrms).to(x.dtype)) * weight


def _layer_rms_norm_fused(x, weight, eps):
    """forward_ref.py:131-133: PyTorch's fused RMSNorm."""
    return F.rms_norm(x, (x.shape[-1],), weight=weight, eps=eps)


def _layer_rope(x, cos, sin):
    """forward_ref.py:43-47: rotate-half RoPE in fp32, cast back."""
    x32 = x.float()
    return (x32 * cos[None, None].float() + _rotate_half(x32) * sin[None, None].float()).to(
        x.dtype)


def _llama3_decoder_layer(rms_norm, x, input_norm_weight, q_weight, k_weight, v_weight,
                          o_weight, post_norm_weight, gate_weight, up_weight, down_weight,
                          cos, sin, eps=1e-5):
    """One Llama-3 decoder layer, restating
    src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:53-117: RMSNorm ->
    Q/K/V projections -> RoPE on q and k -> causal GQA attention (kv heads repeated
    over each query group) -> output projection -> residual -> RMSNorm -> SwiGLU MLP
    (silu in fp32, one rounding) -> residual. Weights in nn.Linear [out, in]
    orientation; head counts from q_out // head_dim and kv_out // head_dim."""
    batch, tokens, hidden = x.shape
    head_dim = cos.shape[-1]
    n_heads = q_weight.shape[0] // head_dim
    n_kv_heads = k_weight.shape[0] // head_dim
    if q_weight.shape[0] % head_dim or k_weight.shape[0] % head_dim:
        raise ValueError("q_out and kv_out must be whole multiples of head_dim")
    if n_heads % n_kv_heads:
        raise ValueError(f"GQA needs n_heads divisible by n_kv_heads, got {n_heads} and "
                         f"{n_kv_heads}")
    h = rms_norm(x, input_norm_weight, eps)
    q = F.linear(h, q_weight).view(batch, tokens, n_heads, head_dim).transpose(1, 2)
    k = F.linear(h, k_weight).view(batch, tokens, n_kv_heads, head_dim).transpose(1, 2)
    v = F.linear(h, v_weight).view(batch, tokens, n_kv_heads, head_dim).transpose(1, 2)
    q = _layer_rope(q, cos, sin)
    k = _layer_rope(k, cos, sin)
    repeat = n_heads // n_kv_heads
    if repeat > 1:
        k = k.repeat_interleave(repeat, dim=1)
        v = v.repeat_interleave(repeat, dim=1)
    attn = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    attn = attn.transpose(1, 2).reshape(batch, tokens, n_heads * head_dim)
    x = x + F.linear(attn, o_weight)
    h = rms_norm(x, post_norm_weight, eps)
    gate = F.linear(h, gate_weight)
    up = F.linear(h, up_weight)
    act = (F.silu(gate.float()) * up.float()).to(h.dtype)
    return x + F.linear(act, down_weight)


def llama3_decoder_layer_forward_ref(*args, **kwargs):
    """The definition, norms spelled out in primitives (forward_ref.py:136-142)."""
    return _llama3_decoder_layer(_layer_rms_norm, *args, **kwargs)


def llama3_decoder_layer_runtime_ref(*args, **kwargs):
    """The same layer with PyTorch's fused RMSNorm, timed as the eager baseline
    (forward_ref.py:145-152)."""
    return _llama3_decoder_layer(_layer_rms_norm_fused, *args, **kwargs)


FORWARDS = {
    "softmax_forward_ref": softmax_forward_ref,
    "rmsnorm_forward_ref": rmsnorm_forward_ref,
    "rmsnorm_runtime_ref": rmsnorm_runtime_ref,
    "fused_add_rms_norm_forward_ref": fused_add_rms_norm_forward_ref,
    "fused_add_rms_norm_runtime_ref": fused_add_rms_norm_runtime_ref,
    "layernorm_forward_ref": layernorm_forward_ref,
    "layernorm_runtime_ref": layernorm_runtime_ref,
    "swiglu_forward_ref": swiglu_forward_ref,
    "rope_forward_ref": rope_forward_ref,
    "causal_attention_forward_ref": causal_attention_forward_ref,
    "causal_attention_runtime_ref": causal_attention_runtime_ref,
    "causal_attention_gqa_forward_ref": causal_attention_gqa_forward_ref,
    "causal_attention_gqa_runtime_ref": causal_attention_gqa_runtime_ref,
    "llama3_attention_forward_ref": llama3_attention_forward_ref,
    "llama3_attention_runtime_ref": llama3_attention_runtime_ref,
    "cross_entropy_forward_ref": cross_entropy_forward_ref,
    "fused_linear_cross_entropy_forward_ref": fused_linear_cross_entropy_forward_ref,
    "llama3_decoder_layer_forward_ref": llama3_decoder_layer_forward_ref,
    "llama3_decoder_layer_runtime_ref": llama3_decoder_layer_runtime_ref,
}
