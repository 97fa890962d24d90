"""Binding and verification wiring on CPU with pure-torch stand-in pairs
(follows the reference's TestBind / TestVerify, tests/test_opdecl_torch.py:143-209)."""

import pytest
import torch

from evograd_amd import decls
from evograd_amd.bind import backward_inactive_kwargs, bind, lookup_pair
from evograd_amd.harness import saved_bytes, saved_state_report
from evograd_amd.opdecl import Workload
from evograd_amd.inputs import make_case_inputs
from oracle.oracle import oracle
from oracle.verify import check_tensor, verify

from tests import stub_pairs

CPU_CASES = (Workload(dims=dict(rows=8, hidden=64), dtype="float32"),
             Workload(dims=dict(rows=17, hidden=128), dtype="bfloat16"))


@pytest.fixture(autouse=True)
def _reset_sabotage():
    for k in stub_pairs.SABOTAGE:
        stub_pairs.SABOTAGE[k] = False
    yield
    for k in stub_pairs.SABOTAGE:
        stub_pairs.SABOTAGE[k] = False


def test_verify_passes_a_correct_pair():
    rep = verify(decls.RMSNORM, stub_pairs, device="cpu", workloads=CPU_CASES)
    assert rep.ok, rep.failures()
    assert [c.name for c in rep.cases[0].checks] == ["y", "dx", "dweight"]


@pytest.mark.parametrize("switch,bad", [("wrong_dweight", {"dweight"}), ("wrong_forward", {"y"})])
def test_verify_names_exactly_the_sabotaged_output(switch, bad):
    stub_pairs.SABOTAGE[switch] = True
    rep = verify(decls.RMSNORM, stub_pairs, device="cpu", workloads=CPU_CASES[:1])
    assert not rep.ok
    failing = {c.name for c in rep.cases[0].checks if not c.ok}
    assert failing == bad


def test_scalar_saved_state_is_allowed():
    stub_pairs.SABOTAGE["scalar_saved"] = True
    rep = verify(decls.RMSNORM, stub_pairs, device="cpu", workloads=CPU_CASES[:1])
    assert rep.ok, rep.failures()
    fn = bind(decls.RMSNORM, stub_pairs)
    x = torch.randn(4, 16, requires_grad=True)
    w = torch.ones(16, requires_grad=True)
    fn(x, w).sum().backward()
    assert x.grad is not None and w.grad is not None


def test_bind_matches_autograd_and_routes_none():
    inputs = make_case_inputs(decls.RMSNORM, CPU_CASES[0], "cpu")
    fn = bind(decls.RMSNORM, stub_pairs)
    x = inputs["x"].clone().requires_grad_(True)
    w = inputs["weight"].clone().requires_grad_(True)
    y = fn(x, w, eps=inputs["eps"])
    gx, gw = torch.autograd.grad(y, (x, w), inputs["dy"])
    y_ref, g_ref = oracle(decls.RMSNORM, inputs)
    assert torch.allclose(y, y_ref, atol=1e-6)
    assert torch.allclose(gx, g_ref["dx"], atol=1e-5) and torch.allclose(gw, g_ref["dweight"], atol=1e-5)
    with pytest.raises(TypeError):
        fn(x)  # missing Active arg
    with pytest.raises(TypeError):
        fn(x, w, bogus=1)
    with pytest.raises(TypeError):
        fn(x, w, 1e-5, 3)


def test_lookup_pair_and_inactive_kwargs():
    fwd, bwd = lookup_pair(decls.SOFTMAX, stub_pairs)
    assert fwd is stub_pairs.softmax_forward_with_saved
    assert backward_inactive_kwargs(decls.SOFTMAX, bwd, {}) == {}
    _, rbwd = lookup_pair(decls.RMSNORM, stub_pairs)
    assert backward_inactive_kwargs(decls.RMSNORM, rbwd, {"eps": 1e-6}) == {"eps": 1e-6}
    with pytest.raises(AttributeError):
        lookup_pair(decls.SWIGLU, stub_pairs)


def test_check_tensor_shape_and_dtype():
    a = torch.zeros(3, 4)
    assert check_tensor("y", a, a.clone(), 1e-5, 1e-5).ok
    assert not check_tensor("y", a, torch.zeros(4, 3), 1e-5, 1e-5).ok
    assert not check_tensor("y", a.double(), a, 1e-5, 1e-5).ok
    assert not check_tensor("y", 3.0, a, 1e-5, 1e-5).ok
    assert not check_tensor("y", a + 1e-3, a, 1e-5, 1e-5).ok


def test_saved_state_accounting():
    x = torch.randn(8, 16)
    w = torch.randn(16)
    y, saved = stub_pairs.rmsnorm_forward_with_saved(x, w)
    assert saved_bytes(saved) == 8 * 16 * 4 + 16 * 4 + 8 * 4
    rep = saved_state_report(saved, {"x": x, "weight": w})
    assert rep["retained_input_bytes"] == 8 * 16 * 4 + 16 * 4
    assert rep["new_storage_bytes"] == 8 * 4
    assert rep["logical_saved_bytes"] == saved_bytes(saved)


def test_input_guard_names_a_mutated_or_reshaped_input():
    from evograd_amd.harness import check_inputs, record_inputs

    values = {"x": torch.randn(4, 8), "weight": torch.randn(8), "eps": 1e-5}
    records = record_inputs(values, may_overwrite=("weight",))
    check_inputs(values, records, "pair")
    values["weight"].mul_(2)  # declared overwritable: contents exempt
    check_inputs(values, records, "pair")
    values["x"][1, 2] += 1
    with pytest.raises(RuntimeError, match="'x' was written to"):
        check_inputs(values, records, "pair")
    values = {"x": torch.randn(4, 8)}
    records = record_inputs(values)
    values["x"] = values["x"].t()
    with pytest.raises(RuntimeError, match="'x' changed"):
        check_inputs(values, records, "pair")
    values = {"weight": torch.randn(8)}
    records = record_inputs(values, may_overwrite=("weight",))
    values["weight"] = torch.randn(9)[1:]  # same shape, other storage offset
    with pytest.raises(RuntimeError, match="'weight' changed"):
        check_inputs(values, records, "pair")
