"""Shape dispatch between two autograd-pair programs (the reference's wire format).

Restates the dispatcher that src/evograd/dispatch.py:98-180 emits, so that a
small-shape and a large-shape HIP program can ship behind one pair:

* the route is computed from the arguments' shapes: every declared tensor
  argument binds its shape tokens to dims (integer tokens must match, a token
  bound twice must agree), the declaration's ``regime_feature`` maps those dims
  to a float, and the route is 0 (small program) below the threshold, 1 (large)
  at or above it (dispatch.py:138-159);
* the forward returns ``(output, (route, *saved))``: the saved state is prefixed
  by a plain integer route tag, which carries no tensor bytes (dispatch.py:162-167);
* the backward pops the tag and calls the same program's backward with the rest
  of the saved state and any further arguments (dispatch.py:170-173).

``ShapeDispatch`` builds such a pair in-process from two loaded modules;
``emit_dispatcher`` writes the same logic as a standalone module that loads the
two programs from files, as the reference's ``_emit_dispatcher`` does.
"""

from __future__ import annotations

import importlib.util
from pathlib import Path
from types import SimpleNamespace

from .opdecl import OpDecl


def _lookup(module, generic: str, prefixed: str):
    value = getattr(module, generic, None)
    return value if value is not None else getattr(module, prefixed)


def shape_dims(op: OpDecl, args: tuple, kwargs: dict) -> dict:
    """Dims bound by the declared tensor arguments' shapes (dispatch.py:139-157)."""
    dims: dict = {}
    for index, declared in enumerate(op.args):
        shape = getattr(declared, "shape", None)
        if shape is None:
            continue
        if index < len(args):
            value = args[index]
        elif declared.name in kwargs:
            value = kwargs[declared.name]
        else:
            raise TypeError(f"missing required argument {declared.name!r}")
        tokens = [part.strip() for part in shape[1:-1].split(",") if part.strip()]
        if len(tokens) != value.dim():
            raise ValueError(f"{declared.name} rank mismatch: {tuple(value.shape)} vs {shape}")
        for token, actual in zip(tokens, value.shape):
            if token.isdigit():
                if int(token) != int(actual):
                    raise ValueError(f"{declared.name} fixed dimension {token} != {actual}")
            elif token in dims and dims[token] != int(actual):
                raise ValueError(f"inconsistent dimension {token}: {dims[token]} != {actual}")
            else:
                dims[token] = int(actual)
    return dims


def route_for(op: OpDecl, threshold: float, args: tuple, kwargs: dict) -> int:
    """0 for the small-shape program, 1 for the large one (dispatch.py:158-159)."""
    if op.regime_feature is None:
        raise ValueError(f"{op.name}: declaration has no regime_feature to dispatch on")
    feature = float(op.regime_feature(SimpleNamespace(dims=shape_dims(op, args, kwargs))))
    return 0 if feature < threshold else 1


class ShapeDispatch:
    """An autograd pair that routes each call to ``small`` or ``large``.

    The object exposes ``forward_with_saved`` / ``backward_from_saved`` and the
    prefixed ``<op>_forward_with_saved`` / ``<op>_backward_from_saved``, so
    ``lookup_pair`` finds it like any candidate module. ``threshold`` defaults to
    the declaration's ``regime_split``.
    """

    def __init__(self, op: OpDecl, small, large, threshold: float | None = None):
        if threshold is None:
            threshold = op.regime_split
        if threshold is None:
            raise ValueError(f"{op.name}: no threshold and no regime_split")
        self.op = op
        self.threshold = float(threshold)
        self.programs = (small, large)
        setattr(self, op.forward_fn_name, self.forward_with_saved)
        setattr(self, op.backward_fn_name, self.backward_from_saved)

    def forward_with_saved(self, *args, **kwargs):
        route = route_for(self.op, self.threshold, args, kwargs)
        forward = _lookup(self.programs[route], "forward_with_saved", self.op.forward_fn_name)
        output, saved = forward(*args, **kwargs)
        saved = tuple(saved) if isinstance(saved, (tuple, list)) else (saved,)
        return output, (route, *saved)

    def backward_from_saved(self, dout, saved_tensors, *args, **kwargs):
        route, *saved = tuple(saved_tensors)
        backward = _lookup(self.programs[int(route)], "backward_from_saved",
                           self.op.backward_fn_name)
        return backward(dout, tuple(saved), *args, **kwargs)


_TEMPLATE = '''"""Shape dispatcher for {name}, written by evograd_amd.dispatch.emit_dispatcher.

Routes at regime_feature < {threshold!r} to the small-shape program, else to the
large one. Saved state is prefixed by a plain integer route tag, which
contributes no tensor-memory bytes.
"""
import importlib.util as _ilu

from evograd_amd.decls import get_op as _get_op
from evograd_amd.dispatch import ShapeDispatch as _ShapeDispatch

_SMALL_PATH = {small!r}
_LARGE_PATH = {large!r}


def _load(label, path):
    spec = _ilu.spec_from_file_location("evograd_amd_dispatch_" + label, path)
    module = _ilu.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


_PAIR = _ShapeDispatch(_get_op({name!r}), _load("small", _SMALL_PATH), _load("large", _LARGE_PATH),
                       {threshold!r})
{forward_fn} = _PAIR.forward_with_saved
{backward_fn} = _PAIR.backward_from_saved
'''


def emit_dispatcher(op: OpDecl, small_path, large_path, threshold: float | None,
                    output) -> Path:
    """Write a standalone dispatcher module (the reference's _emit_dispatcher)."""
    if threshold is None:
        threshold = op.regime_split
    output = Path(output)
    output.parent.mkdir(parents=True, exist_ok=True)
    output.write_text(
        _TEMPLATE.format(name=op.name, threshold=float(threshold),
                         small=str(Path(small_path).resolve()),
                         large=str(Path(large_path).resolve()),
                         forward_fn=op.forward_fn_name, backward_fn=op.backward_fn_name),
        encoding="utf-8",
    )
    return output


def load_module(path):
    """Import a module from a file path (for emitted dispatchers)."""
    spec = importlib.util.spec_from_file_location(Path(path).stem, str(path))
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module
