"""The oracle against the golden fixtures (CPU): numpy fp64 forwards and
finite-difference gradients written independently of torch (tests/golden/
make_golden.py). The oracle's restated forwards widen to fp32, so the bound is
fp32's."""

import pytest
import torch

from evograd_amd import decls
from oracle.oracle import oracle
from tests.golden_cases import OPS, TABLE_ARGS, assert_close, case_inputs

torch.set_grad_enabled(True)


@pytest.mark.parametrize("name", OPS)
def test_oracle_matches_golden(name):
    op = decls.get_op(name)
    inputs, expected, grads = case_inputs(name, torch.float64, "cpu")
    y, g = oracle(op, inputs, use_reference_dtype=False)
    assert_close(f"{name}.{op.output.name}", y, expected, 1e-5, 1e-5)
    for gname, ref in grads.items():
        assert_close(f"{name}.{gname}", g[gname], ref, 1e-4, 1e-5)


def test_golden_fixtures_are_bf16_exact_and_cover_edge_cases():
    for name in OPS:
        inputs, _, _ = case_inputs(name, torch.float64, "cpu")
        for k, v in inputs.items():
            if torch.is_tensor(v) and v.is_floating_point() and k not in TABLE_ARGS.get(name, ()):
                assert torch.equal(v, v.bfloat16().double()), (name, k)
    # an ignored row in both losses
    assert -100 in case_inputs("cross_entropy", torch.float64, "cpu")[0]["target"].tolist()
    assert -100 in case_inputs("fused_linear_cross_entropy", torch.float64,
                               "cpu")[0]["target"].tolist()
