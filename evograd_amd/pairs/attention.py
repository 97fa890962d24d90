"""Causal attention pair on gfx950 (bf16/fp16 MFMA).

Replaces F.scaled_dot_product_attention(q, k, v, is_causal=True) as used at
src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:107, with q, k and v
of one shape [B, H, S, D] (the ``causal_attention`` declaration). Saved state:
``(q, k, v, o, lse)``: the three inputs and the output (no new storage beyond o)
plus the fp32 logsumexp [B, H, S] of the scaled, masked scores, from which the
backward recomputes P. Grouped k, v (fewer heads than q) are the
``causal_attention_gqa`` pair's.
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


def check_operands(q, k, v) -> None:
    """dtype and head_dim rules of the attention entry points (MHA and GQA): fp32,
    bf16 or fp16, an even head_dim up to 128. bf16/fp16 at head_dim 64 or 128 run on
    the MFMA kernels, every other case on the library's generic fp32 kernels."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError(f"attention expects 4-d [B, heads, S, D] tensors; got "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if (q.dtype not in (torch.float32, torch.bfloat16, torch.float16) or k.dtype != q.dtype
            or v.dtype != q.dtype):
        raise TypeError(f"attention supports float32/bfloat16/float16, got "
                        f"{q.dtype}/{k.dtype}/{v.dtype}")
    D = q.shape[-1]
    if D < 2 or D > 128 or D % 2:
        raise ValueError(f"head_dim must be even and at most 128, got {D}")


def causal_attention_forward_with_saved(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    _lib.require_gpu("causal_attention_forward_with_saved", q, k, v)
    check_operands(q, k, v)
    if not (q.shape == k.shape == v.shape):
        raise ValueError(f"causal_attention: q, k, v must share [B, H, S, D]; got "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)} "
                         "(grouped k, v: causal_attention_gqa)")
    q, k, v = (as_contiguous(n, t) for n, t in (("q", q), ("k", k), ("v", v)))
    B, H, S, D = q.shape
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    _lib.call("eg_attn_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(lse),
              B, H, S, D, 1.0 / math.sqrt(D), tag(q.dtype), _lib.stream_of(q))
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
    _lib.call("eg_attn_bwd", _lib.ptr(do), _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o),
              _lib.ptr(lse), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws),
              B, H, S, D, 1.0 / math.sqrt(D), tag(q.dtype), _lib.stream_of(q))
    return dq, dk, dv
