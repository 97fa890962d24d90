"""LayerNorm pair for few rows (the small-shape program of the layernorm dispatcher).

The same operator as ``evograd_amd.pairs.layernorm`` (layernorm_forward_ref,
src/evograd/ops/level1/layernorm/forward_ref.py:6-23; gradients declared at
layernorm/__init__.py:124-171) with the same forward kernel and saved state
``(x, weight, mean, rstd)``. Its backward is the faster of the library's two for
the shape: up to ONE_LAUNCH_MAX_ROWS rows ``eg_layernorm_bwd_small`` (one launch,
no workspace: dweight and dbias summed per column directly from dy, x and the row
statistics while dx is formed per row), above that the ring backward of
``evograd_amd.pairs.layernorm``. Measured on MI355X (bf16, cache flushed, ring +
column sums / one launch, us): hidden 1024: 64 rows 9.7 / 6.2, 512 rows 11.4 / 11.3,
768 rows 12.6 / 14.6; hidden 4096: 64 rows 11.7 / 7.4, 384 rows 14.0 / 12.2, 512 rows
14.7 / 14.7, 768 rows 15.7 / 19.7; hidden 8192: 512 rows 26.4 / 19.8, 1024 rows
33.1 / 34.7 (see ``rmsnorm_small``).
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
from evograd_amd.pairs import layernorm as _ring
from evograd_amd.pairs._util import as_contiguous, tag
from evograd_amd.pairs.layernorm import layernorm_forward_with_saved  # noqa: F401  (same forward)

# Rows up to which the one-launch backward is the faster one (see above).
ONE_LAUNCH_MAX_ROWS = 512


def layernorm_backward_from_saved(dy: torch.Tensor, saved, eps: float = 1e-5):
    x, weight, mean, rstd = saved
    if x.dim() == 2 and x.shape[0] > ONE_LAUNCH_MAX_ROWS:
        return _ring.layernorm_backward_from_saved(dy, saved, eps)
    _lib.require_gpu("layernorm_backward_from_saved", dy, x, weight, mean, rstd)
    if dy.shape != x.shape or dy.dtype != x.dtype:
        raise ValueError("layernorm: dy must match x in shape and dtype")
    dy = as_contiguous("dy", dy)
    rows, hidden = x.shape
    dx = torch.empty_like(x)
    dweight = torch.empty_like(weight)
    dbias = torch.empty_like(weight)
    _lib.call("eg_layernorm_bwd_small", _lib.ptr(dy), _lib.ptr(x), _lib.ptr(weight),
              _lib.ptr(mean), _lib.ptr(rstd), _lib.ptr(dx), _lib.ptr(dweight), _lib.ptr(dbias),
              rows, hidden, tag(x.dtype), _lib.stream_of(x))
    return dx, dweight, dbias
