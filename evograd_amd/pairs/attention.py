"""Causal attention pair on gfx950 (bf16/fp16 MFMA).

Replaces F.scaled_dot_product_attention(q, k, v, is_causal=True) as used at
src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:107. Saved state:
``(q, k, v, o, lse)``: the three inputs and the output (no new storage beyond o)
plus the fp32 logsumexp [B, H, S] of the scaled, masked scores, from which the
backward recomputes P.

k and v may have fewer heads than q (grouped-query attention, H a multiple of
Hkv): query head h attends with kv head h // (H // Hkv), which is the reference's
repeat_interleave of k and v (forward_ref.py:101-105) without the copies; dk and
dv come back with k's and v's shapes, summed over each group.
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from ._util import as_contiguous, tag, workspace


def _check(q, k, v):
    ok = (q.dim() == 4 and k.dim() == 4 and k.shape == v.shape and k.shape[0] == q.shape[0]
          and k.shape[2:] == q.shape[2:] and k.shape[1] > 0 and q.shape[1] % k.shape[1] == 0)
    if not ok:
        raise ValueError(f"attention expects q [B, H, S, D] and k, v [B, Hkv, S, D] with H a "
                         f"multiple of Hkv; got {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError(f"attention supports bfloat16/float16 only, got {q.dtype}")
    if q.shape[-1] not in (64, 128):
        raise ValueError(f"head_dim must be 64 or 128, got {q.shape[-1]}")


def causal_attention_forward_with_saved(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    _lib.require_gpu("causal_attention_forward_with_saved", q, k, v)
    _check(q, k, v)
    q, k, v = (as_contiguous(n, t) for n, t in (("q", q), ("k", k), ("v", v)))
    B, H, S, D = q.shape
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    _lib.call("eg_attn_gqa_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o),
              _lib.ptr(lse), B, H, k.shape[1], S, D, 1.0 / math.sqrt(D), tag(q.dtype),
              _lib.stream_of(q))
    return o, (q, k, v, o, lse)


def causal_attention_backward_from_saved(do: torch.Tensor, saved):
    q, k, v, o, lse = saved
    _lib.require_gpu("causal_attention_backward_from_saved", do, q, k, v, o, lse)
    if do.shape != o.shape or do.dtype != o.dtype:
        raise ValueError("attention: do must match o in shape and dtype")
    do = as_contiguous("do", do)
    B, H, S, D = q.shape
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = workspace(_lib.query("eg_attn_workspace_bytes", B, H, S, D), q.device)
    _lib.call("eg_attn_gqa_bwd", _lib.ptr(do), _lib.ptr(q), _lib.ptr(k), _lib.ptr(v),
              _lib.ptr(o), _lib.ptr(lse), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws),
              B, H, k.shape[1], S, D, 1.0 / math.sqrt(D), tag(q.dtype), _lib.stream_of(q))
    return dq, dk, dv
