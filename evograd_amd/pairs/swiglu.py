"""SwiGLU pair on gfx950.

Replaces swiglu_forward_ref (src/evograd/ops/level1/swiglu/forward_ref.py:6-9)
and the backward declared at swiglu/__init__.py:70-73. Saved state: ``(a, b)``,
the inputs themselves; the sigmoid is recomputed in the backward.

The declaration allows the backward to write da over a and db over b
(``backward_may_overwrite``, swiglu/__init__.py:89-96). ``INPLACE_BACKWARD``
turns that on; it is off by default so the saved inputs stay readable.
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
from evograd_amd.pairs._util import as_contiguous, check_same, tag

INPLACE_BACKWARD = False


def swiglu_forward_with_saved(a: torch.Tensor, b: torch.Tensor):
    _lib.require_gpu("swiglu_forward_with_saved", a, b)
    if a.shape != b.shape:
        raise ValueError(f"a and b must have the same shape, got {a.shape} and {b.shape}")
    check_same("swiglu", a, b)
    a = as_contiguous("a", a)
    b = as_contiguous("b", b)
    c = torch.empty_like(a)
    _lib.call("eg_swiglu_fwd", _lib.ptr(a), _lib.ptr(b), _lib.ptr(c), a.numel(), tag(a.dtype),
              _lib.stream_of(a))
    return c, (a, b)


def swiglu_backward_from_saved(dc: torch.Tensor, saved):
    a, b = saved
    _lib.require_gpu("swiglu_backward_from_saved", dc, a, b)
    if dc.shape != a.shape or dc.dtype != a.dtype:
        raise ValueError("swiglu: dc must match a in shape and dtype")
    dc = as_contiguous("dc", dc)
    if INPLACE_BACKWARD:
        da, db = a, b
    else:
        da, db = torch.empty_like(a), torch.empty_like(b)
    _lib.call("eg_swiglu_bwd", _lib.ptr(dc), _lib.ptr(a), _lib.ptr(b), _lib.ptr(da), _lib.ptr(db),
              a.numel(), tag(a.dtype), _lib.stream_of(a))
    return da, db
