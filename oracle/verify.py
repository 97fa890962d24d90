"""Correctness gate: a pair module against the autograd oracle (test infrastructure only).

Restates src/evograd/opdecl/verify.py:20-160: per workload, build the seeded
inputs, run the oracle, run the module's forward and backward, and check the
output and every gradient for shape, dtype and ``allclose(atol + rtol*|ref|)``.
"""

from __future__ import annotations

import traceback
from dataclasses import dataclass

import torch

from evograd_amd.bind import backward_inactive_kwargs, lookup_pair
from evograd_amd.opdecl import OpDecl, Workload

from evograd_amd.inputs import make_case_inputs
from .oracle import oracle


@dataclass(frozen=True)
class TensorCheck:
    name: str
    ok: bool
    max_abs_err: float
    atol: float
    rtol: float
    actual_shape: tuple = ()
    expected_shape: tuple = ()
    actual_dtype: str = ""
    expected_dtype: str = ""


@dataclass(frozen=True)
class CaseResult:
    dims: dict
    dtype: str
    checks: tuple = ()
    error: str | None = None

    @property
    def ok(self) -> bool:
        return self.error is None and all(c.ok for c in self.checks)


@dataclass(frozen=True)
class VerifyReport:
    op_name: str
    cases: tuple

    @property
    def ok(self) -> bool:
        return bool(self.cases) and all(c.ok for c in self.cases)

    def failures(self) -> list:
        out = []
        for c in self.cases:
            if c.error:
                out.append(f"{c.dims}|{c.dtype}: {c.error.strip().splitlines()[-1]}")
            for t in c.checks:
                if not t.ok:
                    out.append(f"{c.dims}|{c.dtype}: {t.name} max_abs_err={t.max_abs_err:.3g} "
                               f"atol={t.atol} rtol={t.rtol} shape {t.actual_shape} vs "
                               f"{t.expected_shape} dtype {t.actual_dtype} vs {t.expected_dtype}")
        return out

    def to_dict(self) -> dict:
        return {
            "op": self.op_name,
            "ok": self.ok,
            "cases": [
                {"dims": c.dims, "dtype": c.dtype, "ok": c.ok, "error": c.error,
                 "checks": [t.__dict__ | {"actual_shape": list(t.actual_shape),
                                          "expected_shape": list(t.expected_shape)}
                            for t in c.checks]}
                for c in self.cases
            ],
        }


def check_tensor(name: str, actual, expected, atol: float, rtol: float) -> TensorCheck:
    """verify.py:85-115."""
    if not torch.is_tensor(actual):
        return TensorCheck(name, False, float("inf"), atol, rtol,
                           expected_shape=tuple(expected.shape),
                           actual_dtype=type(actual).__name__, expected_dtype=str(expected.dtype))
    same_shape = tuple(actual.shape) == tuple(expected.shape)
    same_dtype = actual.dtype == expected.dtype
    if same_shape:
        a, e = actual.float(), expected.float().to(actual.device)
        max_abs = (a - e).abs().max().item() if a.numel() else 0.0
        values_ok = bool(torch.allclose(a, e, atol=atol, rtol=rtol))
    else:
        max_abs, values_ok = float("inf"), False
    return TensorCheck(name, bool(same_shape and same_dtype and values_ok), max_abs, atol, rtol,
                       tuple(actual.shape), tuple(expected.shape), str(actual.dtype),
                       str(expected.dtype))


def run_case(op: OpDecl, module, workload: Workload, device: str) -> CaseResult:
    """verify.py:118-143."""
    dims, dtype = dict(workload.dims), workload.dtype
    try:
        inputs = make_case_inputs(op, workload, device=device)
        y_ref, ref_grads = oracle(op, inputs)
        fwd, bwd = lookup_pair(op, module)
        positional = [inputs.get(a.name, getattr(a, "default", None)) for a in op.args]
        y, saved = fwd(*positional)
        kwargs = backward_inactive_kwargs(op, bwd, inputs)
        grads = bwd(inputs[op.upstream_grad_name], saved, **kwargs)
        grads = (grads,) if torch.is_tensor(grads) else tuple(grads)
        atol, rtol = op.tolerance_for(workload, op.output.name)
        checks = [check_tensor(op.output.name, y, y_ref, atol, rtol)]
        if len(grads) != len(op.grad_names()):
            raise ValueError(f"backward returned {len(grads)} gradients, contract requires "
                             f"{len(op.grad_names())}: {op.grad_names()}")
        for name, grad in zip(op.grad_names(), grads):
            atol, rtol = op.tolerance_for(workload, name)
            checks.append(check_tensor(name, grad, ref_grads[name], atol, rtol))
        return CaseResult(dims=dims, dtype=dtype, checks=tuple(checks))
    except Exception:
        return CaseResult(dims=dims, dtype=dtype, error=traceback.format_exc())


def verify(op: OpDecl, module, device: str = "cuda", workloads=None) -> VerifyReport:
    """verify.py:146-160; defaults to the declaration's correctness workloads."""
    selected = workloads if workloads is not None else op.correctness
    return VerifyReport(op.name, tuple(run_case(op, module, w, device) for w in selected))
