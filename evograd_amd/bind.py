"""Turn an autograd pair into a differentiable callable.

Contract (the reference's src/evograd/opdecl/bind.py:28-140, which every caller
of a candidate relies on):

* a pair module exposes ``forward_with_saved`` / ``backward_from_saved``, or the
  op-prefixed ``<op>_forward_with_saved`` / ``<op>_backward_from_saved``; the
  generic name wins when both exist;
* ``forward_with_saved(*declared args) -> (y, saved)``, where ``saved`` may mix
  tensors and plain values;
* ``backward_from_saved(dy, saved, **scalars) -> grads`` in ``op.grad_names()``
  order; a scalar Inactive argument is passed again only when the backward's
  signature names it (or takes ``**kwargs``);
* the bound callable returns one gradient slot per declared argument, ``None``
  for every Inactive one.

Design: the declaration is compiled once into a :class:`CallPlan` (argument
order, scalar defaults, gradient slots). One module-level
``torch.autograd.Function`` serves every bound pair; the pair and its plan ride
into it as the first, non-tensor argument. Saved state is split into the tensor
list autograd keeps (``save_for_backward``) and a mask of which positions held
tensors, so the backward gets back exactly the tuple the forward built.
"""

from __future__ import annotations

import inspect
from dataclasses import dataclass

import torch

from .opdecl import Active, OpDecl

_GENERIC = ("forward_with_saved", "backward_from_saved")


def _first_attribute(module, names: tuple):
    for name in names:
        candidate = getattr(module, name, None)
        if candidate is None:
            continue
        if not callable(candidate):
            raise TypeError(f"{name} in {getattr(module, '__name__', module)!r} is a "
                            f"{type(candidate).__name__}, not a function")
        return candidate
    raise AttributeError(f"{getattr(module, '__name__', module)!r} has no "
                         f"{' / '.join(names)}")


def lookup_pair(op: OpDecl, module):
    """``(forward, backward)`` of a pair module, generic names before prefixed ones."""
    prefixed = (op.forward_fn_name, op.backward_fn_name)
    return tuple(_first_attribute(module, (g, p)) for g, p in zip(_GENERIC, prefixed))


def _keyword_names(fn):
    """Names ``fn`` accepts as keywords, or None when it takes ``**kwargs``."""
    names = set()
    for param in inspect.signature(fn).parameters.values():
        if param.kind is inspect.Parameter.VAR_KEYWORD:
            return None
        if param.kind in (inspect.Parameter.POSITIONAL_OR_KEYWORD,
                          inspect.Parameter.KEYWORD_ONLY):
            names.add(param.name)
    return frozenset(names)


def backward_inactive_kwargs(op: OpDecl, bwd, values: dict) -> dict:
    """The scalar Inactive arguments to pass to ``bwd`` again: the call's value, else
    the declared default, for each scalar the backward's signature can take."""
    accepted = _keyword_names(bwd)
    scalars = {a.name: values.get(a.name, a.default) for a in op.scalar_inactive_args()}
    if accepted is None:
        return scalars
    return {name: value for name, value in scalars.items() if name in accepted}


@dataclass(frozen=True)
class CallPlan:
    """How a call of ``op`` maps onto its declared arguments and gradient slots."""

    op: OpDecl
    names: tuple          # declared argument names, in order
    defaults: dict        # scalar Inactive arguments that may be omitted -> default
    grad_slots: tuple     # for each name of op.grad_names(): its argument index
    scalar_names: tuple   # scalar Inactive arguments, in order

    @classmethod
    def of(cls, op: OpDecl) -> "CallPlan":
        names = tuple(a.name for a in op.args)
        index_of_grad = {a.grad_name: i for i, a in enumerate(op.args) if isinstance(a, Active)}
        defaults = {a.name: a.default for a in op.scalar_inactive_args() if a.default is not None}
        return cls(op, names, defaults, tuple(index_of_grad[g] for g in op.grad_names()),
                   tuple(a.name for a in op.scalar_inactive_args()))

    def arrange(self, args: tuple, kwargs: dict, fill_defaults: bool = True) -> dict:
        """``{name: value}`` for a call, in declared order; TypeError on a bad call."""
        label = f"{self.op.name}()"
        if len(args) > len(self.names):
            raise TypeError(f"{label} takes {len(self.names)} arguments "
                            f"({', '.join(self.names)}), {len(args)} were given")
        given = dict(zip(self.names, args))
        for key, value in kwargs.items():
            if key not in self.names:
                raise TypeError(f"{label} has no argument {key!r}")
            if key in given:
                raise TypeError(f"{label} got {key!r} both by position and by keyword")
            given[key] = value
        ordered = {}
        for name in self.names:
            if name in given:
                ordered[name] = given[name]
            elif fill_defaults and name in self.defaults:
                ordered[name] = self.defaults[name]
            elif fill_defaults:
                raise TypeError(f"{label} needs argument {name!r}")
        return ordered

    def scatter(self, grads) -> list:
        """Gradients in ``op.grad_names()`` order -> one slot per declared argument."""
        grads = (grads,) if torch.is_tensor(grads) else tuple(grads)
        if len(grads) != len(self.grad_slots):
            raise ValueError(f"{self.op.name}: the backward gave {len(grads)} gradient(s); "
                             f"the declaration wants {len(self.grad_slots)} "
                             f"({', '.join(self.op.grad_names())})")
        slots = [None] * len(self.names)
        for index, grad in zip(self.grad_slots, grads):
            slots[index] = grad
        return slots


@dataclass(frozen=True)
class _Binding:
    plan: CallPlan
    forward: object
    backward: object
    scalars_for_backward: tuple   # scalar names the backward accepts


class _PairFunction(torch.autograd.Function):
    """Autograd node of a bound pair; ``binding`` is a :class:`_Binding`."""

    @staticmethod
    def forward(ctx, binding, *args):
        y, saved = binding.forward(*args)
        saved = tuple(saved) if isinstance(saved, (tuple, list)) else (saved,)
        mask = tuple(torch.is_tensor(item) for item in saved)
        ctx.save_for_backward(*(item for item, is_t in zip(saved, mask) if is_t))
        ctx.plain = tuple(None if is_t else item for item, is_t in zip(saved, mask))
        ctx.mask = mask
        ctx.binding = binding
        by_name = dict(zip(binding.plan.names, args))
        ctx.scalars = {n: by_name[n] for n in binding.scalars_for_backward}
        return y

    @staticmethod
    def backward(ctx, dy):
        tensors = iter(ctx.saved_tensors)
        saved = tuple(next(tensors) if is_t else plain for is_t, plain in zip(ctx.mask, ctx.plain))
        binding = ctx.binding
        grads = binding.backward(dy.contiguous(), saved, **ctx.scalars)
        return (None, *binding.plan.scatter(grads))


def bind(op: OpDecl, module):
    """A callable ``fn(*declared args, **by name) -> y`` whose backward is the pair's."""
    fwd, bwd = lookup_pair(op, module)
    plan = CallPlan.of(op)
    accepted = backward_inactive_kwargs(op, bwd, {})
    binding = _Binding(plan, fwd, bwd, tuple(n for n in plan.scalar_names if n in accepted))

    def call(*args, **kwargs):
        return _PairFunction.apply(binding, *plan.arrange(args, kwargs).values())

    call.__name__ = call.__qualname__ = f"{op.name}_bound"
    call.plan = plan
    return call
