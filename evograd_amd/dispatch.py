"""Two autograd-pair programs behind one pair, chosen by the call's shapes.

Wire format (the reference's emitted dispatcher, src/evograd/dispatch.py:98-180,
which a saved dispatcher module and its callers agree on):

* the declaration's ``regime_feature`` maps the dims bound by the tensor
  arguments' shapes to a float; below the threshold the call goes to program 0
  (small shapes), at or above it to program 1;
* the forward returns ``(y, (route, *saved))``: a plain ``int`` tag first, so the
  tag adds no tensor bytes to the saved state;
* the backward takes the tag off and hands the rest to the same program.

Design: the argument binding is :class:`evograd_amd.bind.CallPlan`'s (so a call
binds the same way it would through ``bind``); each program's pair is resolved
once, when the dispatcher is built; the shape-token unification sets each dim
by its first binding and compares every later one against it.
``emit_dispatcher`` writes a module file that rebuilds the same object from the
two program files, so the pair can be handed to any tool that loads a candidate
from a path.
"""

from __future__ import annotations

import importlib.util
from pathlib import Path
from types import SimpleNamespace

from .bind import CallPlan, lookup_pair
from .opdecl import OpDecl, shape_tokens

PACKAGE_ROOT = Path(__file__).resolve().parents[1]


def shape_dims(op: OpDecl, args: tuple, kwargs: dict) -> dict:
    """The symbolic dims that the call's tensor arguments fix, e.g. {"rows": 3}."""
    given = CallPlan.of(op).arrange(args, kwargs, fill_defaults=False)
    dims: dict = {}
    for declared in op.args:
        tokens = shape_tokens(getattr(declared, "shape", None))
        if tokens is None:
            continue
        if declared.name not in given:
            raise TypeError(f"{op.name}: shape dispatch needs tensor argument {declared.name!r}")
        sizes = tuple(int(s) for s in given[declared.name].shape)
        if len(sizes) != len(tokens):
            raise ValueError(f"{op.name}: {declared.name} is {len(sizes)}-d {sizes}, "
                             f"declared {declared.shape}")
        for token, size in zip(tokens, sizes):
            expected = int(token) if token.isdigit() else dims.setdefault(token, size)
            if expected != size:
                raise ValueError(f"{op.name}: {declared.name} has {token} = {size}, "
                                 f"the call already fixed it at {expected}")
    return dims


def route_for(op: OpDecl, threshold: float, args: tuple, kwargs: dict) -> int:
    """0 (small-shape program) when the regime feature is below ``threshold``, else 1."""
    if op.regime_feature is None:
        raise ValueError(f"{op.name}: the declaration defines no regime_feature")
    feature = float(op.regime_feature(SimpleNamespace(dims=shape_dims(op, args, kwargs))))
    return int(feature >= threshold)


class ShapeDispatch:
    """A pair (generic and ``<op>_`` names) that routes each call to ``small`` or
    ``large``; ``threshold`` defaults to the declaration's ``regime_split``."""

    def __init__(self, op: OpDecl, small, large, threshold: float | None = None):
        threshold = op.regime_split if threshold is None else threshold
        if threshold is None:
            raise ValueError(f"{op.name}: give a threshold (the declaration has no "
                             "regime_split)")
        self.op = op
        self.threshold = float(threshold)
        self.programs = (small, large)
        self._pairs = tuple(lookup_pair(op, program) for program in self.programs)
        setattr(self, op.forward_fn_name, self.forward_with_saved)
        setattr(self, op.backward_fn_name, self.backward_from_saved)

    def forward_with_saved(self, *args, **kwargs):
        route = route_for(self.op, self.threshold, args, kwargs)
        y, saved = self._pairs[route][0](*args, **kwargs)
        rest = tuple(saved) if isinstance(saved, (tuple, list)) else (saved,)
        return y, (route,) + rest

    def backward_from_saved(self, dy, saved, *args, **kwargs):
        route, rest = int(saved[0]), tuple(saved[1:])
        return self._pairs[route][1](dy, rest, *args, **kwargs)


def load_module(path, prefix: str = "evograd_candidate_"):
    """Execute a module file as a top-level module named ``prefix + stem`` (how
    evograd's verify and bench commands load a candidate)."""
    path = Path(path)
    spec = importlib.util.spec_from_file_location(prefix + path.stem, str(path))
    if spec is None or spec.loader is None:
        raise ImportError(f"cannot load a module from {path}")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


_MODULE_SOURCE = '''"""{name}: shape-dispatched autograd pair (written by evograd_amd.dispatch).

Calls whose regime feature is below {threshold!r} run {small_name}, the others
{large_name}; the saved state starts with the route as a plain int.
"""
import sys as _sys

if {root!r} not in _sys.path:
    _sys.path.insert(0, {root!r})

from evograd_amd.decls import get_op as _get_op
from evograd_amd.dispatch import ShapeDispatch as _ShapeDispatch, load_module as _load_module

_DISPATCH = _ShapeDispatch(
    _get_op({name!r}),
    _load_module({small!r}, "evograd_dispatch_small_"),
    _load_module({large!r}, "evograd_dispatch_large_"),
    {threshold!r},
)
{forward_fn} = _DISPATCH.forward_with_saved
{backward_fn} = _DISPATCH.backward_from_saved
'''


def emit_dispatcher(op: OpDecl, small_path, large_path, threshold: float | None,
                    output) -> Path:
    """Write a loadable module file holding a :class:`ShapeDispatch` over two program
    files (absolute paths are recorded, so the file works from any directory)."""
    threshold = op.regime_split if threshold is None else threshold
    small, large = (Path(p).resolve() for p in (small_path, large_path))
    output = Path(output)
    output.parent.mkdir(parents=True, exist_ok=True)
    output.write_text(_MODULE_SOURCE.format(
        name=op.name, threshold=float(threshold), root=str(PACKAGE_ROOT),
        small=str(small), large=str(large), small_name=small.name, large_name=large.name,
        forward_fn=op.forward_fn_name, backward_fn=op.backward_fn_name), encoding="utf-8")
    return output
