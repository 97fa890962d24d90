"""RMSNorm pair for few rows (the small-shape program of the rmsnorm dispatcher).

The same operator as ``evograd_amd.pairs.rmsnorm`` (rmsnorm_forward_ref,
src/evograd/ops/level1/rmsnorm/forward_ref.py:6-21, backward declared at
rmsnorm/__init__.py:85-86) with the same forward kernel and saved state
``(x, weight, rstd)``. Its backward is the faster of the library's two for the
shape: up to ONE_LAUNCH_MAX_ROWS rows ``eg_rmsnorm_bwd_small`` (one launch, no
workspace: dweight summed per column directly from dy, x and rstd while dx is
formed per row), above that the ring backward of ``evograd_amd.pairs.rmsnorm``
(ring plus column sum). The dispatcher sends this program the shapes under 4096
rows (the reference's small regime, src/evograd/opdecl/models.py:306).

Measured on MI355X (bf16, cache flushed before each call, both backwards through
the C ABI; ring + column sum / one launch, us): hidden 1024: 64 rows 9.6 / 6.2,
512 rows 10.7 / 9.4, 1024 rows 12.8 / 14.2; hidden 4096: 64 rows 11.0 / 7.2,
384 rows 12.4 / 10.4, 512 rows 12.6 / 13.0, 1024 rows 14.8 / 22.1; hidden 8192:
512 rows 20.0 / 18.6, 768 rows 20.6 / 25.3. The one launch reads dy and x twice
(by rows for dx, by columns for dweight), which from about 768 rows on costs more
than the ring's second launch.
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
from evograd_amd.pairs import rmsnorm as _ring
from evograd_amd.pairs._util import as_contiguous, tag
from evograd_amd.pairs.rmsnorm import rmsnorm_forward_with_saved  # noqa: F401  (same forward)

# Rows up to which the one-launch backward is the faster one (see above).
ONE_LAUNCH_MAX_ROWS = 512


def rmsnorm_backward_from_saved(dy: torch.Tensor, saved, eps: float = 1e-5):
    x, weight, rstd = saved
    if x.dim() == 2 and x.shape[0] > ONE_LAUNCH_MAX_ROWS:
        return _ring.rmsnorm_backward_from_saved(dy, saved, eps)
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
