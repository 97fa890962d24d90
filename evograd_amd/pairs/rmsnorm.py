"""RMSNorm pair on gfx950.

Replaces rmsnorm_forward_ref (src/evograd/ops/level1/rmsnorm/forward_ref.py:6-21)
and its autograd backward (rmsnorm/__init__.py:85-86). Saved state:
``(x, weight, rstd)`` where x and weight are the inputs themselves (no new
storage) and rstd is fp32 [rows], 4 bytes per row.
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


def _check(x, weight):
    if x.dim() != 2:
        raise ValueError(f"rmsnorm expects x [rows, hidden], got {tuple(x.shape)}")
    if weight.dim() != 1 or weight.shape[0] != x.shape[1]:
        raise ValueError("weight must be 1D with length hidden")
    check_same("rmsnorm", x, weight)


def rmsnorm_forward_with_saved(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5):
    _lib.require_gpu("rmsnorm_forward_with_saved", x, weight)
    _check(x, weight)
    x = as_contiguous("x", x)
    weight = as_contiguous("weight", weight)
    rows, hidden = x.shape
    y = torch.empty_like(x)
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
    _lib.call("eg_rmsnorm_fwd", _lib.ptr(x), _lib.ptr(weight), _lib.ptr(y), _lib.ptr(rstd),
              rows, hidden, float(eps), tag(x.dtype), _lib.stream_of(x))
    return y, (x, weight, rstd)


def rmsnorm_backward_from_saved(dy: torch.Tensor, saved, eps: float = 1e-5):
    x, weight, rstd = saved
    _lib.require_gpu("rmsnorm_backward_from_saved", dy, x, weight, rstd)
    if dy.shape != x.shape or dy.dtype != x.dtype:
        raise ValueError("rmsnorm: dy must match x in shape and dtype")
    dy = as_contiguous("dy", dy)
    rows, hidden = x.shape
    dx = torch.empty_like(x)
    dweight = torch.empty_like(weight)
    ws = workspace(_lib.query("eg_rmsnorm_workspace_bytes", rows, hidden), x.device)
    _lib.call("eg_rmsnorm_bwd", _lib.ptr(dy), _lib.ptr(x), _lib.ptr(weight), _lib.ptr(rstd),
              _lib.ptr(dx), _lib.ptr(dweight), _lib.ptr(ws), rows, hidden, tag(x.dtype),
              _lib.stream_of(x))
    return dx, dweight
