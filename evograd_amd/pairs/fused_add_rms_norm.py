"""Fused residual-add + RMSNorm pair on gfx950.

Replaces fused_add_rms_norm_forward_ref
(src/evograd/ops/level2/fused_add_rms_norm/forward_ref.py:6-16) and its autograd
backward (dx, dr, dweight; fused_add_rms_norm/__init__.py:76-122). The sum
s = x + r is formed in fp32 inside the kernels and never stored. Saved state:
``(x, r, weight, rstd)``: the inputs themselves (no new storage) plus fp32 rstd
[rows]. The backward forms s again from x and r, which reads the same bytes a
saved s would and stores nothing row-sized.

dx and dr are the same gradient (the gradient through s); the kernel writes it
once and both slots return that tensor.
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


def _check(x, r, weight):
    if x.dim() != 2:
        raise ValueError(f"fused_add_rms_norm expects x [rows, cols], got {tuple(x.shape)}")
    if r.shape != x.shape:
        raise ValueError("fused_add_rms_norm: r must have x's shape")
    if weight.dim() != 1 or weight.shape[0] != x.shape[1]:
        raise ValueError("weight must be 1D with length cols")
    check_same("fused_add_rms_norm", x, r, weight)


def fused_add_rms_norm_forward_with_saved(x: torch.Tensor, r: torch.Tensor,
                                          weight: torch.Tensor, eps: float = 1e-6):
    _lib.require_gpu("fused_add_rms_norm_forward_with_saved", x, r, weight)
    _check(x, r, weight)
    x = as_contiguous("x", x)
    r = as_contiguous("r", r)
    weight = as_contiguous("weight", weight)
    rows, cols = x.shape
    out = torch.empty_like(x)
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
    _lib.call("eg_fused_add_rmsnorm_fwd", _lib.ptr(x), _lib.ptr(r), _lib.ptr(weight),
              _lib.ptr(out), _lib.ptr(rstd), rows, cols, float(eps), tag(x.dtype),
              _lib.stream_of(x))
    return out, (x, r, weight, rstd)


def fused_add_rms_norm_backward_from_saved(dout: torch.Tensor, saved, eps: float = 1e-6):
    x, r, weight, rstd = saved
    _lib.require_gpu("fused_add_rms_norm_backward_from_saved", dout, x, r, weight, rstd)
    if dout.shape != x.shape or dout.dtype != x.dtype:
        raise ValueError("fused_add_rms_norm: dout must match x in shape and dtype")
    dout = as_contiguous("dout", dout)
    rows, cols = x.shape
    ds = torch.empty_like(x)
    dweight = torch.empty_like(weight)
    ws = workspace(_lib.query("eg_rmsnorm_workspace_bytes", rows, cols), x.device)
    _lib.call("eg_fused_add_rmsnorm_bwd", _lib.ptr(dout), _lib.ptr(x), _lib.ptr(r),
              _lib.ptr(weight), _lib.ptr(rstd), _lib.ptr(ds), _lib.ptr(dweight), _lib.ptr(ws),
              rows, cols, tag(x.dtype), _lib.stream_of(x))
    return ds, ds, dweight
