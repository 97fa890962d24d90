"""The declaration contract: naming rules, tolerances, shapes, validation
(mirrors the reference's tests/test_opdecl.py coverage of activity.py)."""

import pytest

from evograd_amd import decls
from evograd_amd.opdecl import Active, Inactive, Workload, bind_shape, declare_op


def test_naming_rules():
    op = decls.RMSNORM
    assert op.forward_fn_name == "rmsnorm_forward_with_saved"
    assert op.backward_fn_name == "rmsnorm_backward_from_saved"
    assert op.grad_names() == ("dx", "dweight")
    assert op.upstream_grad_name == "dy"
    assert [a.name for a in op.scalar_inactive_args()] == ["eps"]
    assert decls.SWIGLU.upstream_grad_name == "dc"
    assert decls.SWIGLU.grad_names() == ("da", "db")
    assert decls.LAYERNORM.grad_names() == ("dx", "dweight", "dbias")
    assert decls.ROPE.grad_names() == ("dx",)
    assert [a.name for a in decls.ROPE.tensor_inactive_args()] == ["cos", "sin"]
    assert decls.CAUSAL_ATTENTION.upstream_grad_name == "do"
    assert decls.CAUSAL_ATTENTION.grad_names() == ("dq", "dk", "dv")


def test_grad_override_and_order():
    op = declare_op(
        name="toy", forward="m:f", dims=("n",),
        args=(Active("x", "[n]"), Active("pair_bias", "[n]", grad="d_pair_bias")),
        output=Active("out", "[n]"), forward_semantics="", backward_semantics="",
        grad_order=("d_pair_bias", "dx"), tolerances={"float32": (1e-5, 1e-5)},
    )
    assert op.grad_names() == ("d_pair_bias", "dx")
    assert op.upstream_grad_name == "dout"


def test_tolerances_match_the_gate():
    w = Workload(dims=dict(rows=4, cols=8), dtype="bfloat16")
    for op in decls.OPS.values():
        for name in (op.output.name, *op.grad_names()):
            if "bfloat16" in op.tolerances:
                expect = (2e-2, 2e-2)
                if op.name == "cross_entropy" and name == "dlogits":
                    expect = (2e-2 / (4 * 8), 2e-2)  # atol scaled to the entry size
                if op.name == "fused_linear_cross_entropy":
                    continue  # its own dims; checked below
                if op.name == "llama3_decoder_layer":
                    # the reference's own block-level gate, with its multipliers
                    expect = (5e-2 * (1.5 if name in ("dk_weight", "dv_weight",
                                                       "ddown_weight") else 1.0), 2e-2)
                assert op.tolerance_for(w, name) == pytest.approx(expect)
    wf = Workload(dims=dict(rows=8, hidden=64, vocab=512), dtype="bfloat16")
    flce = decls.FUSED_LINEAR_CROSS_ENTROPY
    assert flce.tolerance_for(wf, "loss") == (2e-2, 2e-2)
    assert flce.tolerance_for(wf, "dx") == pytest.approx((2e-2 / 8, 2e-2))
    assert flce.tolerance_for(wf, "dweight") == pytest.approx((2e-2 / 512, 2e-2))
    w32 = Workload(dims=dict(rows=4, cols=8), dtype="float32")
    assert decls.SOFTMAX.tolerance_for(w32, "dx") == (1e-5, 1e-5)
    override = Workload(dims=dict(rows=4, cols=8), dtype="float32", atol=1.0, rtol=2.0)
    assert decls.SOFTMAX.tolerance_for(override, "y") == (1.0, 2.0)


def test_bind_shape():
    assert bind_shape("[B, 1, N]", {"B": 2, "N": 128}) == (2, 1, 128)
    assert bind_shape("[]", {}) == ()
    with pytest.raises(ValueError):
        bind_shape("[B, M]", {"B": 2})
    with pytest.raises(ValueError):
        bind_shape("B, M", {"B": 2, "M": 3})


def test_memory_inputs():
    assert decls.ROPE.memory_input_names() == ("x",)
    assert decls.RMSNORM.memory_input_names() == ("x", "weight")
    assert decls.CAUSAL_ATTENTION.memory_input_names() == ("q", "k", "v")


def test_validation_rejects_bad_declarations():
    base = dict(name="bad", forward="m:f", dims=("n",), output=Active("y", "[n]"),
                forward_semantics="", backward_semantics="", tolerances={"float32": (1, 1)})
    with pytest.raises(ValueError):
        declare_op(args=(Active("x", "[n]"), Active("x", "[n]")), **base)
    with pytest.raises(ValueError):
        declare_op(args=(Inactive("eps", default=1e-5),), **base)
    with pytest.raises(ValueError):
        declare_op(args=(Active("x", "[m]"),), **base)
    with pytest.raises(ValueError):
        declare_op(args=(Active("x", "[n]"),), backward_may_overwrite=("z",), **base)
    with pytest.raises(ValueError):
        declare_op(args=(Active("x", "[n]"),),
                   correctness=(Workload(dims={"n": 4}, dtype="float16"),), **base)


BASELINE_OPS = ("softmax", "rmsnorm", "layernorm", "swiglu", "rope", "causal_attention")


def test_baseline_workloads_present():
    labels = {name: [w for w in decls.get_op(name).benchmark if w.label == "baseline"]
              for name in BASELINE_OPS}
    assert all(labels.values()), labels
    # the operators beyond the six above carry the reference's own timed workload
    farn = decls.FUSED_ADD_RMS_NORM.benchmark[0]
    assert farn.dims == {"rows": 16384, "cols": 4096} and farn.dtype == "bfloat16"
    assert decls.RMSNORM.benchmark[0].dims == {"rows": 16384, "hidden": 4096}
    assert decls.RMSNORM.benchmark[0].extra["eps"] == 1e-6
    assert decls.SWIGLU.benchmark[0].dims == {"rows": 16384, "cols": 14336}
    assert decls.CAUSAL_ATTENTION.benchmark[0].dims == {"B": 4, "H": 32, "S": 4096, "D": 128}


def test_get_op_unknown():
    with pytest.raises(KeyError):
        decls.get_op("nope")
    assert decls.get_op("softmax") is decls.SOFTMAX
