"""Grouped-query causal attention pair on gfx950 (k, v with fewer heads than q).

Replaces the repeat_interleave of k and v followed by the causal SDPA in
src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:101-107 without the
copies: query head h attends with kv head h // (H // Hkv), read in place. dk and
dv come back with k's and v's shapes, each the sum over its group of query heads,
accumulated in a fixed order inside one workgroup (no atomics, bitwise
repeatable). Saved state: ``(q, k, v, o, lse)``, lse fp32 [B, H, S]; no
repeated k or v is ever stored.
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
from evograd_amd.pairs.attention import check_operands


def group_size(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> int:
    """Query heads per kv head; raises unless k and v are [B, Hkv, S, D] with Hkv | H."""
    check_operands(q, k, v)
    B, H, S, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[2:] != q.shape[2:]:
        raise ValueError(f"causal_attention_gqa: k and v must be [B, Hkv, S, D] matching q "
                         f"{tuple(q.shape)} in B, S, D; got {tuple(k.shape)}, {tuple(v.shape)}")
    kv_heads = k.shape[1]
    if kv_heads == 0 or H % kv_heads:
        raise ValueError(f"causal_attention_gqa: {H} query heads are not a multiple of "
                         f"{kv_heads} kv heads")
    return H // kv_heads


def causal_attention_gqa_forward_with_saved(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    _lib.require_gpu("causal_attention_gqa_forward_with_saved", q, k, v)
    group_size(q, k, v)
    q, k, v = (as_contiguous(n, t) for n, t in (("q", q), ("k", k), ("v", v)))
    B, H, S, D = q.shape
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    _lib.call("eg_attn_gqa_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o),
              _lib.ptr(lse), B, H, k.shape[1], S, D, 1.0 / math.sqrt(D), tag(q.dtype),
              _lib.stream_of(q))
    return o, (q, k, v, o, lse)


def causal_attention_gqa_backward_from_saved(do: torch.Tensor, saved):
    q, k, v, o, lse = saved
    _lib.require_gpu("causal_attention_gqa_backward_from_saved", do, q, k, v, o, lse)
    if do.shape != o.shape or do.dtype != o.dtype:
        raise ValueError("causal_attention_gqa: do must match o in shape and dtype")
    do = as_contiguous("do", do)
    B, H, S, D = q.shape
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = workspace(_lib.query("eg_attn_gqa_workspace_bytes", B, H, k.shape[1], S, D), q.device)
    _lib.call("eg_attn_gqa_bwd", _lib.ptr(do), _lib.ptr(q), _lib.ptr(k), _lib.ptr(v),
              _lib.ptr(o), _lib.ptr(lse), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws),
              B, H, k.shape[1], S, D, 1.0 / math.sqrt(D), tag(q.dtype), _lib.stream_of(q))
    return dq, dk, dv
