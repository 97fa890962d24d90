"""Half-rotated RoPE pair on gfx950.

Replaces rope_forward_ref (src/evograd/ops/level1/rope/forward_ref.py:28-47) and
the backward declared at rope/__init__.py:124-130. Saved state: ``(cos, sin)``,
the caller's tables (no new storage). The tables may be fp32 or x's dtype; any
other dtype is converted to fp32 once.

``rope_qk_forward_with_saved`` / ``rope_qk_backward_from_saved`` rotate the query
and key tensors of a GQA layer in one launch each way (the tables are read once
per token for both).
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

import torch

from evograd_amd import _lib
from evograd_amd.pairs._util import as_contiguous, tag


def _tables(x, cos, sin):
    if cos.shape != sin.shape or cos.dim() != 2:
        raise ValueError("cos and sin must both be [T, head_dim]")
    if cos.dtype != sin.dtype or cos.dtype not in (torch.float32, x.dtype):
        cos, sin = cos.float(), sin.float()
    return as_contiguous("cos", cos), as_contiguous("sin", sin)


def _check_x(name, x, cos):
    if x.dim() != 4:
        raise ValueError(f"rope expects [batch, heads, tokens, head_dim], got {tuple(x.shape)}")
    if x.shape[-1] % 2:
        raise ValueError(f"rope needs an even head_dim, got {x.shape[-1]}")
    if tuple(cos.shape) != (x.shape[2], x.shape[3]):
        raise ValueError(f"{name}: tables {tuple(cos.shape)} do not match tokens/head_dim of {tuple(x.shape)}")


def _launch(q, k, qo, ko, cos, sin, inverse):
    B, Hq, T, D = q.shape
    Hk = k.shape[1] if k is not None else 0
    _lib.call("eg_rope", _lib.ptr(q), _lib.ptr(k), _lib.ptr(qo), _lib.ptr(ko), _lib.ptr(cos),
              _lib.ptr(sin), B, Hq, Hk, T, D, tag(q.dtype), tag(cos.dtype), int(inverse),
              _lib.stream_of(q))


def rope_forward_with_saved(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    _lib.require_gpu("rope_forward_with_saved", x, cos, sin)
    cos, sin = _tables(x, cos, sin)
    _check_x("rope", x, cos)
    x = as_contiguous("x", x)
    y = torch.empty_like(x)
    _launch(x, None, y, None, cos, sin, inverse=False)
    return y, (cos, sin)


def rope_backward_from_saved(dy: torch.Tensor, saved):
    cos, sin = saved
    _lib.require_gpu("rope_backward_from_saved", dy, cos, sin)
    _check_x("rope", dy, cos)
    dy = as_contiguous("dy", dy)
    dx = torch.empty_like(dy)
    _launch(dy, None, dx, None, cos, sin, inverse=True)
    return dx


def rope_qk_forward_with_saved(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor,
                               sin: torch.Tensor):
    _lib.require_gpu("rope_qk_forward_with_saved", q, k, cos, sin)
    cos, sin = _tables(q, cos, sin)
    _check_x("rope q", q, cos)
    _check_x("rope k", k, cos)
    if q.shape[0] != k.shape[0] or q.shape[2:] != k.shape[2:] or q.dtype != k.dtype:
        raise ValueError("q and k must share batch, tokens, head_dim and dtype")
    q, k = as_contiguous("q", q), as_contiguous("k", k)
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    _launch(q, k, qo, ko, cos, sin, inverse=False)
    return (qo, ko), (cos, sin)


class RopeQK(torch.autograd.Function):
    """The joint q/k pair as an autograd node: ``RopeQK.apply(q, k, cos, sin)`` ->
    ``(q', k')``; the tables get no gradient."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        (qo, ko), saved = rope_qk_forward_with_saved(q, k, cos, sin)
        ctx.save_for_backward(*saved)
        return qo, ko

    @staticmethod
    def backward(ctx, dq_out, dk_out):
        dq, dk = rope_qk_backward_from_saved((dq_out, dk_out), ctx.saved_tensors)
        return dq, dk, None, None


def rope_qk_backward_from_saved(grads, saved):
    dq_out, dk_out = grads
    cos, sin = saved
    _lib.require_gpu("rope_qk_backward_from_saved", dq_out, dk_out, cos, sin)
    _check_x("rope q", dq_out, cos)
    _check_x("rope k", dk_out, cos)
    dq_out, dk_out = as_contiguous("dq", dq_out), as_contiguous("dk", dk_out)
    dq, dk = torch.empty_like(dq_out), torch.empty_like(dk_out)
    _launch(dq_out, dk_out, dq, dk, cos, sin, inverse=True)
    return dq, dk
