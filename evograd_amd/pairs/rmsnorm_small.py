"""RMSNorm pair for few rows (the small-shape program of the rmsnorm dispatcher).

The same operator as ``evograd_amd.pairs.rmsnorm`` (rmsnorm_forward_ref,
src/evograd/ops/level1/rmsnorm/forward_ref.py:6-21, backward declared at
rmsnorm/__init__.py:85-86) with the same forward kernel and saved state
``(x, weight, rstd)``; the backward is ``eg_rmsnorm_bwd_small``: one launch, no
workspace, dweight summed per column directly from dy, x and rstd while dx is
formed per row. Under 4096 rows (the reference's small regime,
src/evograd/opdecl/models.py:306) the ring backward's two latency-bound launches
cost more than this kernel's second read of dy and x, which the device cache
serves at those sizes.
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
from evograd_amd.pairs.rmsnorm import rmsnorm_forward_with_saved  # noqa: F401  (same forward)


def rmsnorm_backward_from_saved(dy: torch.Tensor, saved, eps: float = 1e-5):
    x, weight, rstd = saved
    _lib.require_gpu("rmsnorm_backward_from_saved", dy, x, weight, rstd)
    if dy.shape != x.shape or dy.dtype != x.dtype:
        raise ValueError("rmsnorm: dy must match x in shape and dtype")
    dy = as_contiguous("dy", dy)
    rows, hidden = x.shape
    dx = torch.empty_like(x)
    dweight = torch.empty_like(weight)
    _lib.call("eg_rmsnorm_bwd_small", _lib.ptr(dy), _lib.ptr(x), _lib.ptr(weight),
              _lib.ptr(rstd), _lib.ptr(dx), _lib.ptr(dweight), rows, hidden, tag(x.dtype),
              _lib.stream_of(x))
    return dx, dweight
