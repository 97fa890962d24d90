"""Ground-truth forward and gradients from the declaration (test infrastructure only).

Restates src/evograd/opdecl/oracle.py:22-111: ``requires_grad`` is set on exactly
the Active arguments, the declared forward runs under autograd, and
``torch.autograd.grad`` with the upstream gradient yields the reference
gradients. With ``reference_dtype`` set, floating inputs are widened first and
the results cast back to the dtypes the candidate must return (:70-110).
"""

from __future__ import annotations

import importlib

import torch

from evograd_amd.opdecl import Active, OpDecl


def resolve_callable(path: str):
    """"module:function" -> callable (the reference's importing.resolve_callable)."""
    mod, _, fn = path.partition(":")
    if not mod or not fn:
        raise ValueError(f"expected 'module:function', got {path!r}")
    return getattr(importlib.import_module(mod), fn)


def resolve_forward(op: OpDecl):
    return resolve_callable(op.forward)


def resolve_runtime_forward(op: OpDecl):
    """The forward timed as the eager baseline (oracle.py:22-34)."""
    return resolve_callable(op.runtime_forward or op.forward)


_RUNTIME_CHECKED: set = set()


def check_runtime_forward(op: OpDecl, device: str = "cpu") -> int:
    """Hold the forward timed as the eager baseline (``runtime_forward``) to the
    declared ``forward`` on every correctness workload before anything times it
    (the reference's verify_runtime_forward, src/evograd/opdecl/baselines.py:82-121):
    same shape, same dtype, allclose at the declaration's tolerance. Returns the
    number of workloads checked (0 when the op declares no separate runtime
    forward, so the timed function is the declared one); raises RuntimeError on a
    disagreement."""
    if not op.runtime_forward:
        return 0
    from evograd_amd.inputs import make_case_inputs

    definition, runtime = resolve_forward(op), resolve_runtime_forward(op)
    with torch.no_grad():
        for w in op.correctness:
            inputs = make_case_inputs(op, w, device)
            args = [inputs.get(a.name, getattr(a, "default", None)) for a in op.args]
            want, got = definition(*args), runtime(*args)
            atol, rtol = op.tolerance_for(w, op.output.name)
            if (got.shape != want.shape or got.dtype != want.dtype
                    or not torch.allclose(got.float(), want.float(), atol=atol, rtol=rtol)):
                raise RuntimeError(f"{op.name}: runtime forward {op.runtime_forward} differs "
                                   f"from {op.forward} at {w.dims}/{w.dtype}")
    _RUNTIME_CHECKED.add(op.name)
    return len(op.correctness)


def _promote(value, dtype):
    if torch.is_tensor(value) and value.is_floating_point():
        return value.to(dtype)
    return value


def oracle(op: OpDecl, inputs: dict, dout: torch.Tensor | None = None, *,
           use_reference_dtype: bool = True):
    """Run the forward reference under autograd; return ``(y, grads)``.

    ``grads`` maps gradient names to tensors in ``op.grad_names()`` order.
    """
    fwd = resolve_forward(op)
    ref_dtype = (
        getattr(torch, op.reference_dtype)
        if (op.reference_dtype and use_reference_dtype)
        else None
    )
    positional, leaves, out_dtypes = [], [], {}
    for arg in op.args:
        value = inputs.get(arg.name, getattr(arg, "default", None))
        if value is None:
            raise ValueError(f"{op.name}: missing input {arg.name!r} and no default")
        if isinstance(arg, Active):
            out_dtypes[arg.grad_name] = value.dtype
            if ref_dtype is not None:
                value = _promote(value, ref_dtype)
            value = value.detach().clone().requires_grad_(True)
            leaves.append((arg.grad_name, value))
        elif ref_dtype is not None:
            value = _promote(value, ref_dtype)
        positional.append(value)

    y = fwd(*positional)
    if dout is None:
        dout = inputs[op.upstream_grad_name]
    y_dtype = dout.dtype
    if ref_dtype is not None:
        dout = _promote(dout, ref_dtype)
    grads = torch.autograd.grad(y, [t for _, t in leaves], grad_outputs=dout)
    by_name = {name: g for (name, _), g in zip(leaves, grads)}
    if ref_dtype is not None:
        y = y.to(y_dtype)
        by_name = {n: g.to(out_dtypes[n]) for n, g in by_name.items()}
    return y.detach(), {n: by_name[n].detach() for n in op.grad_names()}
