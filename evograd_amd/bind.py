"""Wrap an autograd pair into a ``torch.autograd.Function``.

Restates src/evograd/opdecl/bind.py:28-140: the declaration drives argument
routing, so ``None`` lands in the gradient slot of every Inactive argument and
the returned gradients are placed by name, never by position guesswork.

A pair module exposes (generic or op-prefixed names):

    forward_with_saved(*declared args)  -> (y, saved)
    backward_from_saved(dy, saved, **scalar inactive args it accepts) -> grads

``saved`` may mix tensors and plain values; tensors go through
``save_for_backward``, plain values ride in a side layout.
"""

from __future__ import annotations

import inspect

import torch

from .opdecl import Active, OpDecl


def lookup_pair(op: OpDecl, module):
    """The module's forward/backward, generic or prefixed names (bind.py:28-47)."""

    def _lookup(generic: str, prefixed: str):
        fn = getattr(module, generic, None)
        if fn is None:
            fn = getattr(module, prefixed, None)
        if fn is None:
            raise AttributeError(
                f"module {getattr(module, '__name__', module)!r} defines neither "
                f"{generic!r} nor {prefixed!r}"
            )
        if not callable(fn):
            raise TypeError(f"attribute {generic!r}/{prefixed!r} is not callable")
        return fn

    return (
        _lookup("forward_with_saved", op.forward_fn_name),
        _lookup("backward_from_saved", op.backward_fn_name),
    )


def backward_inactive_kwargs(op: OpDecl, bwd, values: dict) -> dict:
    """Scalar Inactive args the backward's signature accepts (bind.py:50-59)."""
    params = inspect.signature(bwd).parameters
    accepts_kwargs = any(p.kind is inspect.Parameter.VAR_KEYWORD for p in params.values())
    return {
        c.name: values.get(c.name, c.default)
        for c in op.scalar_inactive_args()
        if c.name in params or accepts_kwargs
    }


def bind(op: OpDecl, module):
    """Return ``fn(*declared args) -> y`` with autograd wired up (bind.py:62-140)."""
    fwd, bwd = lookup_pair(op, module)
    arg_names = [a.name for a in op.args]
    slot_by_grad = {a.grad_name: i for i, a in enumerate(op.args) if isinstance(a, Active)}
    return_names = op.grad_names()

    class _Bound(torch.autograd.Function):
        @staticmethod
        def forward(ctx, *args):
            y, saved = fwd(*args)
            saved = tuple(saved) if isinstance(saved, (tuple, list)) else (saved,)
            tensors, layout = [], []
            for item in saved:
                if torch.is_tensor(item):
                    layout.append(("tensor", len(tensors)))
                    tensors.append(item)
                else:
                    layout.append(("value", item))
            ctx.save_for_backward(*tensors)
            ctx.saved_layout = layout
            ctx.inactive_values = {
                c.name: args[arg_names.index(c.name)] for c in op.scalar_inactive_args()
            }
            return y

        @staticmethod
        def backward(ctx, dout):
            saved = tuple(
                ctx.saved_tensors[payload] if kind == "tensor" else payload
                for kind, payload in ctx.saved_layout
            )
            kwargs = backward_inactive_kwargs(op, bwd, ctx.inactive_values)
            grads = bwd(dout.contiguous(), saved, **kwargs)
            grads = (grads,) if torch.is_tensor(grads) else tuple(grads)
            if len(grads) != len(return_names):
                raise ValueError(
                    f"{op.name}: backward returned {len(grads)} gradients, "
                    f"contract requires {len(return_names)}: {return_names}"
                )
            slots: list = [None] * len(arg_names)
            for name, grad in zip(return_names, grads):
                slots[slot_by_grad[name]] = grad
            return tuple(slots)

    def call(*args, **kwargs):
        if len(args) > len(arg_names):
            raise TypeError(
                f"{op.name}: expected at most {len(arg_names)} positional args, got {len(args)}"
            )
        named = dict(zip(arg_names, args))
        unknown = set(kwargs) - set(arg_names)
        if unknown:
            raise TypeError(f"{op.name}: unexpected keyword arguments {sorted(unknown)}")
        duplicates = set(kwargs) & set(arg_names[: len(args)])
        if duplicates:
            raise TypeError(f"{op.name}: multiple values for arguments {sorted(duplicates)}")
        named.update(kwargs)
        full = []
        for arg in op.args:
            if arg.name in named:
                full.append(named[arg.name])
            elif isinstance(arg, Active) or getattr(arg, "is_tensor", False):
                raise TypeError(f"{op.name}: missing required argument {arg.name!r}")
            elif arg.default is not None:
                full.append(arg.default)
            else:
                raise TypeError(f"{op.name}: missing required argument {arg.name!r}")
        return _Bound.apply(*full)

    call.__name__ = f"{op.name}_autograd"
    call.__qualname__ = call.__name__
    return call
