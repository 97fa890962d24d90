"""No HIP pair changes its inputs: every tensor of a case (declared arguments and the
upstream gradient) keeps its shape, strides, dtype and storage offset and, unless
the declaration lists it in ``backward_may_overwrite`` (SwiGLU's a and b), its
contents, across the forward and across the backward
(src/evograd/bench/fair.py:212-261)."""

import sys

import pytest
import torch

from evograd_amd import PAIR_MODULES, decls, pair_module
from evograd_amd.bind import backward_inactive_kwargs, lookup_pair
from evograd_amd.harness import check_inputs, record_inputs
from evograd_amd.inputs import make_case_inputs

pytestmark = pytest.mark.gpu


def _cases():
    for name in sorted(PAIR_MODULES):
        op = decls.get_op(name)
        for w in (*op.correctness[:3], op.benchmark[0]):
            yield pytest.param(name, w, id=f"{name}-{w.key()}")


@pytest.mark.parametrize("name,w", list(_cases()))
def test_pair_leaves_its_inputs_unchanged(name, w):
    print(f"\n[gpu-inputs] {name} {w.dims} {w.dtype}", flush=True)
    sys.stdout.flush()
    op = decls.get_op(name)
    values = make_case_inputs(op, w, "cuda")
    fwd, bwd = lookup_pair(op, pair_module(name))
    args = [values[a.name] for a in op.args]
    records = record_inputs(values, op.backward_may_overwrite)
    with torch.no_grad():
        y, saved = fwd(*args)
        torch.cuda.synchronize()
        check_inputs(values, records, f"{name} forward")
        kwargs = backward_inactive_kwargs(op, bwd, values)
        grads = bwd(values[op.upstream_grad_name], saved, **kwargs)
        torch.cuda.synchronize()
    check_inputs(values, records, f"{name} backward")
    del y, saved, grads, values, records
    torch.cuda.empty_cache()
