"""layernorm: shape-dispatched pair over this library's two layernorm programs.

Rows below the declaration's regime split (4096, the reference's small/large
boundary for Llama-width operators, src/evograd/opdecl/models.py:306) run
``evograd_amd.pairs.layernorm_small`` (one-launch backward), the others
``evograd_amd.pairs.layernorm`` (the ring backward). The saved state starts with the
route as a plain int, the wire format of the reference's emitted dispatcher
(src/evograd/dispatch.py:98-180).
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

from evograd_amd.decls import LAYERNORM
from evograd_amd.dispatch import ShapeDispatch
from evograd_amd.pairs import layernorm as _large
from evograd_amd.pairs import layernorm_small as _small

_DISPATCH = ShapeDispatch(LAYERNORM, _small, _large)
layernorm_forward_with_saved = _DISPATCH.forward_with_saved
layernorm_backward_from_saved = _DISPATCH.backward_from_saved
