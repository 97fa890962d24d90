"""Shape dispatch wire format (src/evograd/dispatch.py:98-180) on CPU with pure-torch
stand-in pairs: routing by the declaration's regime feature, the integer route tag
prefixed to the saved state, the backward following the tag, shape checks, and the
emitted standalone module."""

import types

import pytest
import torch

from evograd_amd import decls
from evograd_amd.bind import bind, lookup_pair
from evograd_amd.dispatch import ShapeDispatch, emit_dispatcher, load_module, route_for, shape_dims
from evograd_amd.harness import saved_bytes
from evograd_amd.opdecl import Workload
from oracle.verify import verify

from tests import stub_pairs


def _recording(tag, calls):
    """A stub RMSNorm program that records which direction ran under which tag."""
    mod = types.SimpleNamespace()

    def fwd(x, weight, eps=1e-5):
        calls.append((tag, "fwd"))
        return stub_pairs.rmsnorm_forward_with_saved(x, weight, eps)

    def bwd(dy, saved, eps=1e-5):
        calls.append((tag, "bwd"))
        return stub_pairs.rmsnorm_backward_from_saved(dy, saved, eps)

    mod.rmsnorm_forward_with_saved = fwd
    mod.rmsnorm_backward_from_saved = bwd
    return mod


def test_route_follows_regime_feature_and_split():
    op = decls.RMSNORM
    assert op.regime_split == 4096.0
    w = torch.ones(8)
    assert route_for(op, op.regime_split, (torch.zeros(4095, 8), w), {}) == 0
    assert route_for(op, op.regime_split, (torch.zeros(4096, 8), w), {}) == 1
    assert route_for(op, 10.0, (torch.zeros(9, 8),), {"weight": w}) == 0
    assert shape_dims(op, (torch.zeros(3, 8), w), {}) == {"rows": 3, "hidden": 8}
    with pytest.raises(ValueError, match="is 3-d"):
        route_for(op, 10.0, (torch.zeros(3, 8, 1), w), {})
    with pytest.raises(ValueError, match="already fixed it at 8"):
        route_for(op, 10.0, (torch.zeros(3, 8), torch.ones(7)), {})
    with pytest.raises(TypeError, match="needs tensor argument 'weight'"):
        route_for(op, 10.0, (torch.zeros(3, 8),), {})


def test_saved_state_is_prefixed_by_an_int_route_and_backward_follows_it():
    calls = []
    pair = ShapeDispatch(decls.RMSNORM, _recording("small", calls), _recording("large", calls),
                         threshold=16)
    x, w = torch.randn(20, 8), torch.ones(8)
    y, saved = pair.rmsnorm_forward_with_saved(x, w, 1e-5)
    assert saved[0] == 1 and isinstance(saved[0], int)
    assert saved_bytes(saved) == saved_bytes(saved[1:])  # the tag carries no tensor bytes
    pair.rmsnorm_backward_from_saved(torch.randn_like(y), saved, eps=1e-5)
    _, saved_small = pair.rmsnorm_forward_with_saved(x[:4], w, 1e-5)
    pair.rmsnorm_backward_from_saved(torch.randn(4, 8), saved_small, eps=1e-5)
    assert calls == [("large", "fwd"), ("large", "bwd"), ("small", "fwd"), ("small", "bwd")]
    fwd, bwd = lookup_pair(decls.RMSNORM, pair)
    assert fwd == pair.forward_with_saved and bwd == pair.backward_from_saved


def test_dispatched_pair_passes_the_gate_and_binds():
    calls = []
    pair = ShapeDispatch(decls.RMSNORM, _recording("small", calls), _recording("large", calls),
                         threshold=16)
    cases = (Workload(dims=dict(rows=8, hidden=64), dtype="float32"),
             Workload(dims=dict(rows=17, hidden=128), dtype="bfloat16"))
    rep = verify(decls.RMSNORM, pair, device="cpu", workloads=cases)
    assert rep.ok, rep.failures()
    assert {c[0] for c in calls} == {"small", "large"}
    x = torch.randn(5, 16, requires_grad=True)
    w = torch.ones(16, requires_grad=True)
    bind(decls.RMSNORM, pair)(x, w, 1e-5).sum().backward()
    assert x.grad is not None and w.grad is not None


def test_emitted_module_loads_both_programs(tmp_path):
    small = tmp_path / "small.py"
    large = tmp_path / "large.py"
    source = open(stub_pairs.__file__).read()
    small.write_text(source)
    large.write_text(source)
    out = emit_dispatcher(decls.RMSNORM, small, large, 16.0, tmp_path / "dispatch_rmsnorm.py")
    mod = load_module(out)
    x, w = torch.randn(20, 8), torch.ones(8)
    y, saved = mod.rmsnorm_forward_with_saved(x, w, 1e-5)
    assert saved[0] == 1
    ref, _ = stub_pairs.rmsnorm_forward_with_saved(x, w, 1e-5)
    assert torch.equal(y, ref)
    dx, dw = mod.rmsnorm_backward_from_saved(torch.ones_like(y), saved, eps=1e-5)
    assert dx.shape == x.shape and dw.shape == w.shape


def test_every_declaration_carries_the_reference_regime():
    assert decls.SOFTMAX.regime_split == 2048.0
    for name in ("rmsnorm", "layernorm", "swiglu", "fused_add_rms_norm"):
        op = decls.get_op(name)
        assert op.regime_split == 4096.0
        assert op.regime_feature(types.SimpleNamespace(dims={"rows": 7, "hidden": 1, "cols": 1})) == 7.0
    assert decls.ROPE.regime_feature(types.SimpleNamespace(dims={"T": 5})) == 5.0
