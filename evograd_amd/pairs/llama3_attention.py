"""RoPE(q, k) -> grouped causal attention as one pair on gfx950.

Replaces the attention half of the Llama-3 decoder layer,
src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:93-107: q and k
rotated by the half-rotated RoPE (:42-51), k and v repeated over each query
group (:101-105), causal SDPA (:107).

Saved state: ``(q, k, v, o, lse, cos, sin)``. q and k are the caller's
pre-rotation tensors, so the only new storage is o and the fp32 logsumexp
[B, H, S] (plus fp32 copies of the tables when the caller's are not fp32). The
backward rotates q and k again into its workspace; that costs one pass over q
and k, where saving the rotated tensors would keep B*(H + KVH)*S*D more elements
alive between the passes. The forward rotates q inside the attention kernel as it
loads it, and the backward applies the rotation's transpose to dq and dk inside
the kernels before they are stored: the only separate rotation launches are k's
in the forward and q's and k's in the backward.
"""

from __future__ import annotations

if not __package__:
    # Loaded from this file's path as a top-level candidate module (evograd's verify
    # and bench commands load a program that way): put the package root on sys.path.
    import pathlib as _pathlib
    import sys as _sys

    _ROOT = str(_pathlib.Path(__file__).resolve().parents[2])
    if _ROOT not in _sys.path:
        _sys.path.insert(0, _ROOT)

import math

import torch

from evograd_amd import _lib
from evograd_amd.pairs._util import as_contiguous, tag, workspace
from evograd_amd.pairs.attention_gqa import group_size


def _tables(q, cos, sin):
    S, D = q.shape[2], q.shape[3]
    if tuple(cos.shape) != (S, D) or tuple(sin.shape) != (S, D):
        raise ValueError(f"llama3_attention: cos and sin must be [S, D] = [{S}, {D}], got "
                         f"{tuple(cos.shape)}, {tuple(sin.shape)}")
    return (as_contiguous("cos", cos.to(torch.float32)),
            as_contiguous("sin", sin.to(torch.float32)))


def _check_mfma(q):
    """The fused RoPE -> attention kernels are the MFMA ones: bf16/fp16, head_dim 64
    or 128."""
    if q.dtype not in (torch.bfloat16, torch.float16) or q.shape[-1] not in (64, 128):
        raise ValueError(f"llama3_attention: bfloat16/float16 with head_dim 64 or 128, got "
                         f"{q.dtype} at head_dim {q.shape[-1]}")


def llama3_attention_forward_with_saved(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                        cos: torch.Tensor, sin: torch.Tensor):
    _lib.require_gpu("llama3_attention_forward_with_saved", q, k, v, cos, sin)
    group_size(q, k, v)
    _check_mfma(q)
    cos, sin = _tables(q, cos, sin)
    q, k, v = (as_contiguous(n, t) for n, t in (("q", q), ("k", k), ("v", v)))
    B, H, S, D = q.shape
    KVH = k.shape[1]
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    ws = workspace(k.numel() * k.element_size(), q.device)  # the rotated keys
    _lib.call("eg_llama3_attn_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(cos),
              _lib.ptr(sin), _lib.ptr(o), _lib.ptr(lse), _lib.ptr(ws), B, H, KVH, S, D,
              1.0 / math.sqrt(D), tag(q.dtype), _lib.stream_of(q))
    return o, (q, k, v, o, lse, cos, sin)


def llama3_attention_backward_from_saved(do: torch.Tensor, saved):
    q, k, v, o, lse, cos, sin = saved
    _lib.require_gpu("llama3_attention_backward_from_saved", do, q, k, v, o, lse, cos, sin)
    if do.shape != o.shape or do.dtype != o.dtype:
        raise ValueError("llama3_attention: do must match o in shape and dtype")
    do = as_contiguous("do", do)
    B, H, S, D = q.shape
    KVH = k.shape[1]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = workspace(_lib.query("eg_llama3_attn_workspace_bytes", B, H, KVH, S, D), q.device)
    _lib.call("eg_llama3_attn_bwd", _lib.ptr(do), _lib.ptr(q), _lib.ptr(k), _lib.ptr(v),
              _lib.ptr(o), _lib.ptr(lse), _lib.ptr(cos), _lib.ptr(sin), _lib.ptr(dq),
              _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws), B, H, KVH, S, D, 1.0 / math.sqrt(D),
              tag(q.dtype), _lib.stream_of(q))
    return dq, dk, dv
