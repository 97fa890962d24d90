"""Operator declaration contract (torch-free).

Restates the part of src/evograd/opdecl/activity.py that the autograd-pair hot
path consumes: which arguments are differentiable (``Active``) or not
(``Inactive``), symbolic shapes, workloads, per-dtype tolerances and the naming
rules that tie a candidate module's functions and gradients to the declaration.

Naming rules (activity.py:1-20, :301-337):

* an Active input's gradient is ``"d" + name`` unless ``grad`` overrides it;
* the upstream gradient is the output's gradient name (``y`` -> ``dy``);
* backward returns the Active gradients in declaration order unless
  ``grad_order`` overrides it;
* the pair is ``<op>_forward_with_saved`` / ``<op>_backward_from_saved`` (or the
  generic ``forward_with_saved`` / ``backward_from_saved``).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable


@dataclass(frozen=True)
class Active:
    """Differentiable tensor argument (activity.py:28-45)."""

    name: str
    shape: str = "unspecified"
    dtype: str | None = None
    grad: str | None = None
    note: str = ""

    @property
    def grad_name(self) -> str:
        return self.grad if self.grad is not None else f"d{self.name}"


@dataclass(frozen=True)
class Inactive:
    """Non-differentiable argument: a tensor when ``shape`` is set, else a scalar
    whose default is re-passed to the backward as a keyword (activity.py:48-65)."""

    name: str
    shape: str | None = None
    dtype: str | None = None
    default: float | int | None = None
    note: str = ""

    @property
    def is_tensor(self) -> bool:
        return self.shape is not None


def shape_tokens(shape) -> tuple | None:
    """``"[rows, cols]"`` -> ``("rows", "cols")``; None when no shape is declared."""
    if not isinstance(shape, str):
        return None
    text = shape.strip()
    if not (text.startswith("[") and text.endswith("]")):
        return None
    return tuple(t.strip() for t in text[1:-1].split(",") if t.strip())


def bind_shape(shape: str, dims: dict[str, int]) -> tuple[int, ...]:
    """Resolve ``"[rows, cols]"`` against concrete dims (activity.py:84-100)."""
    text = shape.strip()
    if not (text.startswith("[") and text.endswith("]")):
        raise ValueError(f"shape must look like '[A, B]', got {shape!r}")
    body = text[1:-1].strip()
    if not body:
        return ()
    out = []
    for token in body.split(","):
        token = token.strip()
        if token in dims:
            out.append(int(dims[token]))
        elif token.isdigit():
            out.append(int(token))
        else:
            raise ValueError(f"shape dim {token!r} not bound by {sorted(dims)}")
    return tuple(out)


@dataclass(frozen=True)
class Workload:
    """One concrete case: dims, dtype, optional per-case tolerance override and
    a label (activity.py:159-176)."""

    dims: dict
    dtype: str
    atol: float | None = None
    rtol: float | None = None
    label: str = ""
    extra: dict = field(default_factory=dict)

    def key(self) -> str:
        dims = ",".join(f"{k}={v}" for k, v in self.dims.items())
        return f"{self.label or 'case'}[{dims}|{self.dtype}]"


@dataclass(frozen=True)
class OpDecl:
    """Single source of truth for one operator (activity.py:179-570)."""

    name: str
    forward: str
    dims: tuple
    args: tuple
    output: Active
    forward_semantics: str
    backward_semantics: str
    runtime_forward: str | None = None
    reference_dtype: str | None = None
    grad_order: tuple | None = None
    correctness: tuple = ()
    benchmark: tuple = ()
    tolerances: dict = field(default_factory=dict)
    # Per-result (atol, rtol) factors applied to the base tolerance before the hook
    # (activity.py:245, :524-525).
    tolerance_multipliers: dict = field(default_factory=dict)
    tolerance_hook: Callable | None = None
    make_inputs: str | None = None
    memory_inputs: tuple | None = None
    backward_may_overwrite: tuple = ()
    # Shape regimes (activity.py:258-262): regime_feature maps an object with a
    # ``dims`` mapping to a float; a shape dispatcher routes below regime_split to
    # its small-shape program.
    regime_feature: Callable | None = None
    regime_split: float | None = None

    # ---- derived views (activity.py:289-337)
    def active_args(self) -> tuple:
        return tuple(a for a in self.args if isinstance(a, Active))

    def inactive_args(self) -> tuple:
        return tuple(a for a in self.args if isinstance(a, Inactive))

    def tensor_inactive_args(self) -> tuple:
        return tuple(a for a in self.inactive_args() if a.is_tensor)

    def scalar_inactive_args(self) -> tuple:
        return tuple(a for a in self.inactive_args() if not a.is_tensor)

    def grad_names(self) -> tuple:
        default = tuple(a.grad_name for a in self.active_args())
        return self.grad_order if self.grad_order is not None else default

    @property
    def upstream_grad_name(self) -> str:
        return self.output.grad_name

    @property
    def forward_fn_name(self) -> str:
        return f"{self.name}_forward_with_saved"

    @property
    def backward_fn_name(self) -> str:
        return f"{self.name}_backward_from_saved"

    def tolerance_for(self, workload: Workload, result_name: str | None = None) -> tuple:
        """(atol, rtol) for one checked result (activity.py:517-528)."""
        if workload.atol is not None and workload.rtol is not None:
            atol, rtol = workload.atol, workload.rtol
        else:
            atol, rtol = self.tolerances[workload.dtype]
        scale = self.tolerance_multipliers.get(result_name or "", (1.0, 1.0))
        atol, rtol = atol * scale[0], rtol * scale[1]
        if self.tolerance_hook is not None:
            atol, rtol = self.tolerance_hook(workload, result_name, atol, rtol)
        return float(atol), float(rtol)

    def memory_input_names(self) -> tuple:
        """Inputs that count as the op's memory footprint (activity.py:530-535)."""
        if self.memory_inputs is not None:
            return self.memory_inputs
        return tuple(a.name for a in self.args if getattr(a, "shape", None) is not None)

    def validate(self) -> None:
        names = [a.name for a in self.args]
        if len(set(names)) != len(names):
            raise ValueError(f"{self.name}: duplicate argument names {names}")
        if not self.active_args():
            raise ValueError(f"{self.name}: at least one Active argument is required")
        grads = [a.grad_name for a in self.active_args()]
        if self.output.grad_name in names or self.output.name in names:
            raise ValueError(f"{self.name}: output name collides with an argument")
        if self.grad_order is not None and sorted(self.grad_order) != sorted(grads):
            raise ValueError(f"{self.name}: grad_order {self.grad_order} != grads {grads}")
        for arg in self.args:
            shape = getattr(arg, "shape", None)
            if shape is not None and isinstance(arg, (Active, Inactive)) and shape != "unspecified":
                self._validate_shape(arg.name, shape)
        self._validate_shape(self.output.name, self.output.shape)
        for w in (*self.correctness, *self.benchmark):
            missing = set(self.dims) - set(w.dims)
            if missing:
                raise ValueError(f"{self.name}: workload {w.dims} misses dims {sorted(missing)}")
            if w.atol is None and w.dtype not in self.tolerances:
                raise ValueError(f"{self.name}: no tolerance for dtype {w.dtype}")
        unknown = set(self.tolerance_multipliers) - set(self.grad_names())
        if unknown:
            raise ValueError(f"{self.name}: tolerance multipliers name unknown gradients "
                             f"{sorted(unknown)}")
        for name, factors in self.tolerance_multipliers.items():
            if len(factors) != 2 or any(f <= 0 for f in factors):
                raise ValueError(f"{self.name}: tolerance multiplier for {name} must be two "
                                 "positive values")
        for name in self.backward_may_overwrite:
            if name not in [a.name for a in self.active_args()]:
                raise ValueError(f"{self.name}: backward_may_overwrite names non-Active {name!r}")
        if self.regime_feature is not None or self.regime_split is not None:
            # activity.py:463-471
            if not callable(self.regime_feature) or self.regime_split is None:
                raise ValueError(f"{self.name}: shape regimes require callable regime_feature "
                                 "and numeric regime_split")
            if self.regime_split <= 0:
                raise ValueError(f"{self.name}: regime_split must be positive")

    def _validate_shape(self, arg_name: str, shape: str) -> None:
        text = shape.strip()
        if not (text.startswith("[") and text.endswith("]")):
            raise ValueError(f"{self.name}.{arg_name}: bad shape {shape!r}")
        body = text[1:-1].strip()
        if not body:
            return
        for token in body.split(","):
            token = token.strip()
            if token not in self.dims and not token.isdigit():
                raise ValueError(
                    f"{self.name}.{arg_name}: dim {token!r} is neither declared {self.dims} "
                    "nor an integer literal"
                )


def declare_op(**kwargs) -> OpDecl:
    """Build and validate an OpDecl (activity.py:611-682)."""
    for key in ("dims", "args", "correctness", "benchmark", "backward_may_overwrite"):
        if key in kwargs and kwargs[key] is not None:
            kwargs[key] = tuple(kwargs[key])
    if kwargs.get("grad_order") is not None:
        kwargs["grad_order"] = tuple(kwargs["grad_order"])
    if kwargs.get("memory_inputs") is not None:
        kwargs["memory_inputs"] = tuple(kwargs["memory_inputs"])
    op = OpDecl(**kwargs)
    op.validate()
    return op

