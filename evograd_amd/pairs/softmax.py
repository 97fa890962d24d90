"""Row softmax pair on gfx950.

Replaces the eager pair of src/evograd/ops/level1/softmax/forward_ref.py:6-7 with
backward rule softmax/__init__.py:78. Saved state: ``(y,)``, the output itself
(rows*cols elements of x's dtype). Softmax runs over the last dimension; leading
dimensions are flattened into rows.
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


def softmax_forward_with_saved(x: torch.Tensor):
    _lib.require_gpu("softmax_forward_with_saved", x)
    x = as_contiguous("x", x)
    y = torch.empty_like(x)
    cols = x.shape[-1] if x.dim() else 1
    rows = x.numel() // cols if cols else 0
    _lib.call("eg_softmax_fwd", _lib.ptr(x), _lib.ptr(y), rows, cols, tag(x.dtype),
              _lib.stream_of(x))
    return y, (y,)


def softmax_backward_from_saved(dy: torch.Tensor, saved):
    (y,) = saved
    _lib.require_gpu("softmax_backward_from_saved", dy, y)
    if dy.shape != y.shape or dy.dtype != y.dtype:
        raise ValueError(f"softmax: dy {tuple(dy.shape)}/{dy.dtype} vs y {tuple(y.shape)}/{y.dtype}")
    dy = as_contiguous("dy", dy)
    dx = torch.empty_like(y)
    cols = y.shape[-1] if y.dim() else 1
    rows = y.numel() // cols if cols else 0
    _lib.call("eg_softmax_bwd", _lib.ptr(y), _lib.ptr(dy), _lib.ptr(dx), rows, cols,
              tag(y.dtype), _lib.stream_of(y))
    return dx
