"""LayerNorm pair on gfx950.

Replaces layernorm_forward_ref (src/evograd/ops/level1/layernorm/forward_ref.py:6-23)
and its autograd backward (grads dx, dweight, dbias; layernorm/__init__.py:124-171).
Saved state: ``(x, weight, mean, rstd)``: the inputs x and weight (no new storage)
plus fp32 mean and rstd [rows]. bias is not needed by the backward.
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
from evograd_amd.pairs._util import as_contiguous, check_same, tag, workspace


def layernorm_forward_with_saved(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
                                 eps: float = 1e-5):
    _lib.require_gpu("layernorm_forward_with_saved", x, weight, bias)
    if x.dim() != 2:
        raise ValueError(f"layernorm expects x [rows, hidden], got {tuple(x.shape)}")
    if weight.dim() != 1 or bias.dim() != 1 or weight.shape[0] != x.shape[1] or bias.shape[0] != x.shape[1]:
        raise ValueError("weight and bias must be 1D with length hidden")
    check_same("layernorm", x, weight, bias)
    x = as_contiguous("x", x)
    weight = as_contiguous("weight", weight)
    bias = as_contiguous("bias", bias)
    rows, hidden = x.shape
    y = torch.empty_like(x)
    mean = torch.empty(rows, dtype=torch.float32, device=x.device)
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
    _lib.call("eg_layernorm_fwd", _lib.ptr(x), _lib.ptr(weight), _lib.ptr(bias), _lib.ptr(y),
              _lib.ptr(mean), _lib.ptr(rstd), rows, hidden, float(eps), tag(x.dtype),
              _lib.stream_of(x))
    return y, (x, weight, mean, rstd)


def layernorm_backward_from_saved(dy: torch.Tensor, saved, eps: float = 1e-5):
    x, weight, mean, rstd = saved
    _lib.require_gpu("layernorm_backward_from_saved", dy, x, weight, mean, rstd)
    if dy.shape != x.shape or dy.dtype != x.dtype:
        raise ValueError("layernorm: dy must match x in shape and dtype")
    dy = as_contiguous("dy", dy)
    rows, hidden = x.shape
    dx = torch.empty_like(x)
    dweight = torch.empty_like(weight)
    dbias = torch.empty_like(weight)
    ws = workspace(_lib.query("eg_layernorm_workspace_bytes", rows, hidden), x.device)
    _lib.call("eg_layernorm_bwd", _lib.ptr(dy), _lib.ptr(x), _lib.ptr(weight), _lib.ptr(mean),
              _lib.ptr(rstd), _lib.ptr(dx), _lib.ptr(dweight), _lib.ptr(dbias), _lib.ptr(ws),
              rows, hidden, tag(x.dtype), _lib.stream_of(x))
    return dx, dweight, dbias
