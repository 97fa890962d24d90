"""Parity of the HIP pairs with the autograd oracle on the GPU.

Every case runs the reference's gate (restated in oracle/verify.py): identical
seeded inputs, the oracle's forward and gradients, then shape, dtype and
allclose on the output and every gradient at this build's tolerances
(fp32 1e-5/1e-5, fp16 1e-2/1e-2, bf16 2e-2/2e-2; see evograd_amd/decls.py).
The benchmark-size cases run the same gate at full size plus size-independent
properties (bitwise determinism of the two-stage reductions, in-place backward,
joint q/k RoPE == two single launches).
"""

import sys

import pytest
import torch

from evograd_amd import decls, pair_module
from evograd_amd.inputs import make_case_inputs
from oracle.oracle import oracle
from oracle.verify import verify

pytestmark = pytest.mark.gpu

MEMORY_BOUND = ("softmax", "rmsnorm", "layernorm", "swiglu", "rope", "fused_add_rms_norm",
                "cross_entropy")


def _cases(names):
    for name in names:
        for w in decls.get_op(name).correctness:
            yield pytest.param(name, w, id=f"{name}-{w.key()}")


def _run(name, w):
    print(f"\n[gpu-parity] {name} {w.dims} {w.dtype} {w.label}", flush=True)
    sys.stdout.flush()
    rep = verify(decls.get_op(name), pair_module(name), device="cuda", workloads=(w,))
    torch.cuda.synchronize()
    assert rep.ok, "\n".join(rep.failures())
    return rep


@pytest.mark.parametrize("name,w", list(_cases(MEMORY_BOUND)))
def test_memory_bound_correctness_workloads(name, w):
    _run(name, w)


@pytest.mark.parametrize("name", MEMORY_BOUND)
def test_memory_bound_baseline_config(name):
    for w in decls.get_op(name).benchmark:
        _run(name, w)
        torch.cuda.empty_cache()


# Row widths at the edges of the softmax kernels' row configurations: 16-byte packs per
# row (npack) at each boundary of the register-row choices (64 .. 8192 packs of 512-1024
# threads), the 16-bit LDS-row path above 8192 packs and the two-read loop past it; ragged
# widths (a partial last pack) between them.
_SOFTMAX_EDGES = (64, 65, 128, 129, 256, 257, 512, 513, 1000, 1024, 1025, 2048, 2049, 4096,
                  4097, 8192, 8193)


def _softmax_edge_cases():
    from evograd_amd.opdecl import Workload

    for dtype, vec in (("float32", 4), ("bfloat16", 8), ("float16", 8)):
        for npack in _SOFTMAX_EDGES:
            for cols in (npack * vec, npack * vec - 3):
                yield pytest.param(Workload(dims=dict(rows=3, cols=cols), dtype=dtype),
                                   id=f"{dtype}-{cols}")


@pytest.mark.parametrize("w", list(_softmax_edge_cases()))
def test_softmax_row_configuration_edges(w):
    _run("softmax", w)


# Row widths at the edges of the norm kernels' configurations: the one-wave forwards
# (1, 2 and 4 packs per lane), the two-row forward, and the rings of 1024 threads with 2, 4
# and 8 packs per thread (hidden up to 65536 bf16 / 32768 fp32), whole and ragged, at a few
# rows and at more rows than the backward ring has workgroups.
_NORM_EDGES = (("bfloat16", 512), ("bfloat16", 1024), ("bfloat16", 2048), ("bfloat16", 8200),
               ("bfloat16", 16384), ("bfloat16", 16392), ("bfloat16", 32768), ("bfloat16", 65536),
               ("float16", 12288), ("float32", 1024), ("float32", 8192), ("float32", 16384),
               ("float32", 32768), ("float32", 8191))


def _norm_edge_cases():
    from evograd_amd.opdecl import Workload

    for name in ("rmsnorm", "layernorm", "fused_add_rms_norm"):
        width = "cols" if name == "fused_add_rms_norm" else "hidden"
        for dtype, hidden in _NORM_EDGES:
            for rows in (3, 600):
                if rows * hidden > (1 << 22):
                    continue
                yield pytest.param(name, Workload(dims={"rows": rows, width: hidden}, dtype=dtype),
                                   id=f"{name}-{dtype}-{rows}x{hidden}")


@pytest.mark.parametrize("name,w", list(_norm_edge_cases()))
def test_norm_width_edges(name, w):
    _run(name, w)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_softmax_vocab_rows_with_masked_entries(dtype):
    """Rows of -inf entries on the on-chip (LDS) row path, as a causal or padding mask
    gives them: a row whose first half is -inf, a row with -inf scattered through it,
    a finite row, and a row of -inf only (NaN, as torch gives). Forward and backward
    against torch's autograd in fp32, cast back."""
    mod = pair_module("softmax")
    g = torch.Generator(device="cuda").manual_seed(11)
    rows, cols = 4, 100000
    x = torch.randn(rows, cols, device="cuda", generator=g).to(dtype)
    x[0, : cols // 2] = float("-inf")
    x[1, ::7] = float("-inf")
    x[3] = float("-inf")
    dy = torch.randn(rows, cols, device="cuda", generator=g).to(dtype)
    print(f"\n[gpu-parity] softmax masked rows {dtype}", flush=True)
    y, saved = mod.softmax_forward_with_saved(x)
    dx = mod.softmax_backward_from_saved(dy, saved)
    dx = dx[0] if isinstance(dx, tuple) else dx
    xr = x.float().requires_grad_(True)
    yr = torch.softmax(xr, -1)
    (dxr,) = torch.autograd.grad(yr, xr, dy.float())
    torch.cuda.synchronize()
    assert torch.isnan(y[3]).all() and torch.isnan(yr[3]).all()
    torch.testing.assert_close(y[:3].float(), yr[:3].to(dtype).float(), atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(dx[:3].float(), dxr[:3].to(dtype).float(), atol=2e-2, rtol=2e-2)
    assert (y[0, : cols // 2] == 0).all() and (y[1, ::7] == 0).all()


def test_rmsnorm_backward_is_bitwise_deterministic():
    op = decls.RMSNORM
    w = op.benchmark[0]
    inp = make_case_inputs(op, w, "cuda")
    mod = pair_module("rmsnorm")
    _, saved = mod.rmsnorm_forward_with_saved(inp["x"], inp["weight"], inp["eps"])
    a = mod.rmsnorm_backward_from_saved(inp["dy"], saved, eps=inp["eps"])
    b = mod.rmsnorm_backward_from_saved(inp["dy"], saved, eps=inp["eps"])
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_layernorm_backward_is_bitwise_deterministic():
    op = decls.LAYERNORM
    inp = make_case_inputs(op, op.correctness[-3], "cuda")
    mod = pair_module("layernorm")
    _, saved = mod.layernorm_forward_with_saved(inp["x"], inp["weight"], inp["bias"], inp["eps"])
    a = mod.layernorm_backward_from_saved(inp["dy"], saved)
    b = mod.layernorm_backward_from_saved(inp["dy"], saved)
    assert all(torch.equal(x, y) for x, y in zip(a, b))


def test_swiglu_inplace_backward_matches():
    mod = pair_module("swiglu")
    op = decls.SWIGLU
    w = op.correctness[-1]
    inp = make_case_inputs(op, w, "cuda")
    _, saved = mod.swiglu_forward_with_saved(inp["a"], inp["b"])
    ref = mod.swiglu_backward_from_saved(inp["dc"], saved)
    a2, b2 = inp["a"].clone(), inp["b"].clone()
    mod.INPLACE_BACKWARD = True
    try:
        da, db = mod.swiglu_backward_from_saved(inp["dc"], (a2, b2))
    finally:
        mod.INPLACE_BACKWARD = False
    assert da.data_ptr() == a2.data_ptr() and db.data_ptr() == b2.data_ptr()
    assert torch.equal(da, ref[0]) and torch.equal(db, ref[1])


def test_rope_joint_qk_equals_single_launches_and_oracle():
    mod = pair_module("rope")
    w = decls.ROPE.benchmark[0]
    inp = make_case_inputs(decls.ROPE, w, "cuda")
    q = inp["x"]
    torch.manual_seed(1234)
    k = torch.randn((q.shape[0], w.extra["k_heads"], q.shape[2], q.shape[3]), device="cuda",
                    dtype=q.dtype)
    (qo, ko), saved = mod.rope_qk_forward_with_saved(q, k, inp["cos"], inp["sin"])
    qo1, _ = mod.rope_forward_with_saved(q, inp["cos"], inp["sin"])
    ko1, _ = mod.rope_forward_with_saved(k, inp["cos"], inp["sin"])
    assert torch.equal(qo, qo1) and torch.equal(ko, ko1)
    dq, dk = mod.rope_qk_backward_from_saved((inp["dy"], k), saved)
    assert torch.equal(dq, mod.rope_backward_from_saved(inp["dy"], saved))
    yk, gk = oracle(decls.ROPE, {"x": k, "cos": inp["cos"], "sin": inp["sin"], "dy": k})
    assert torch.allclose(ko.float(), yk.float(), atol=2e-2, rtol=2e-2)
    assert torch.allclose(dk.float(), gk["dx"].float(), atol=2e-2, rtol=2e-2)
    # the rotation is orthogonal: per (i, i + half) pair the norm is preserved
    half = q.shape[-1] // 2
    n_in = q.float()[..., :half] ** 2 + q.float()[..., half:] ** 2
    n_out = qo.float()[..., :half] ** 2 + qo.float()[..., half:] ** 2
    assert torch.allclose(n_in, n_out, rtol=2e-2, atol=2e-2)


def test_rope_joint_qk_partial_head_groups():
    """Heads are served in groups of four: q with 6 heads (a full and a partial group)
    and k with 2 (one partial group) in one joint launch equal two single launches and
    the oracle."""
    mod = pair_module("rope")
    g = torch.Generator(device="cpu").manual_seed(99)
    q = torch.randn((2, 6, 33, 128), generator=g).to("cuda", torch.bfloat16)
    k = torch.randn((2, 2, 33, 128), generator=g).to("cuda", torch.bfloat16)
    pos = torch.arange(33, dtype=torch.float32)[:, None]
    inv = 10000.0 ** (-torch.arange(0, 64, dtype=torch.float32) / 64)
    ang = torch.cat([pos * inv, pos * inv], dim=-1)
    cos, sin = ang.cos().cuda(), ang.sin().cuda()
    print("\n[gpu-parity] rope joint q[2,6,33,128] k[2,2,33,128] bf16", flush=True)
    (qo, ko), saved = mod.rope_qk_forward_with_saved(q, k, cos, sin)
    assert torch.equal(qo, mod.rope_forward_with_saved(q, cos, sin)[0])
    assert torch.equal(ko, mod.rope_forward_with_saved(k, cos, sin)[0])
    for x, y in ((q, qo), (k, ko)):
        yr, _ = oracle(decls.ROPE, {"x": x, "cos": cos, "sin": sin, "dy": x})
        assert torch.allclose(y.float(), yr.float(), atol=2e-2, rtol=2e-2)
    dq, dk = mod.rope_qk_backward_from_saved((q, k), saved)
    _, gq = oracle(decls.ROPE, {"x": q, "cos": cos, "sin": sin, "dy": q})
    _, gk = oracle(decls.ROPE, {"x": k, "cos": cos, "sin": sin, "dy": k})
    assert torch.allclose(dq.float(), gq["dx"].float(), atol=2e-2, rtol=2e-2)
    assert torch.allclose(dk.float(), gk["dx"].float(), atol=2e-2, rtol=2e-2)
    # the same pair as an autograd node (the benchmark's autograd-bound step)
    ql, kl = q.detach().requires_grad_(True), k.detach().requires_grad_(True)
    qa, ka = mod.RopeQK.apply(ql, kl, cos, sin)
    assert torch.equal(qa, qo) and torch.equal(ka, ko)
    torch.autograd.backward((qa, ka), (q, k))
    assert torch.equal(ql.grad, dq) and torch.equal(kl.grad, dk)


def test_fused_add_rms_norm_backward_deterministic_and_grads_not_aliased():
    """Bitwise-repeatable backward at the Llama-3-8B size; through the autograd
    binding x.grad and r.grad hold equal values in separate storage (the pair
    returns the single gradient through s for both slots)."""
    from evograd_amd.bind import bind

    op = decls.FUSED_ADD_RMS_NORM
    w = op.benchmark[0]
    print(f"\n[gpu-parity] fused_add_rms_norm determinism {w.dims}", flush=True)
    inp = make_case_inputs(op, w, "cuda")
    mod = pair_module("fused_add_rms_norm")
    _, saved = mod.fused_add_rms_norm_forward_with_saved(inp["x"], inp["r"], inp["weight"],
                                                         inp["eps"])
    a = mod.fused_add_rms_norm_backward_from_saved(inp["dout"], saved, eps=inp["eps"])
    b = mod.fused_add_rms_norm_backward_from_saved(inp["dout"], saved, eps=inp["eps"])
    assert all(torch.equal(p, q) for p, q in zip(a, b))
    small = make_case_inputs(op, decls.FUSED_ADD_RMS_NORM.correctness[-1], "cuda")
    leaves = [small[n].detach().requires_grad_(True) for n in ("x", "r", "weight")]
    y = bind(op, mod)(*leaves, small["eps"])
    y.backward(small["dout"])
    gx, gr = leaves[0].grad, leaves[1].grad
    assert torch.equal(gx, gr)
    assert gx.untyped_storage().data_ptr() != gr.untyped_storage().data_ptr()


def _first_bwd_kernel(bwd, dy, saved, **kw) -> str:
    """Name of the first kernel a backward call launches (the timing hook's label)."""
    from evograd_amd.timing import KernelTimer

    timer = KernelTimer()
    try:
        timer.arm(0)
        bwd(dy, saved, **kw)
        timer.elapsed_ms()
        return timer.label()
    finally:
        timer.close()


@pytest.mark.parametrize("name", ["rmsnorm", "layernorm"])
def test_shape_dispatch_routes_to_two_programs(name):
    """The dispatched pair over two different HIP programs: below the declaration's
    4096-row split the small-shape program (the one-launch backward, norm_bwd_small,
    up to 512 rows, the ring above), at or above it the ring program
    (norm_bwd_ring); both pass the gate, the saved state carries the route tag, and
    each route runs the kernel its program picks for the shape."""
    from evograd_amd import dispatch_module
    from evograd_amd.opdecl import Workload

    op = decls.get_op(name)
    pair = dispatch_module(name)
    fwd = getattr(pair, op.forward_fn_name)
    bwd = getattr(pair, op.backward_fn_name)
    cases = ((Workload(dims=dict(rows=300, hidden=768), dtype="bfloat16"), 0, "norm_bwd_small"),
             (Workload(dims=dict(rows=512, hidden=1000), dtype="float32"), 0, "norm_bwd_small"),
             (Workload(dims=dict(rows=513, hidden=768), dtype="bfloat16"), 0, "norm_bwd_ring"),
             (Workload(dims=dict(rows=1500, hidden=1000), dtype="float32"), 0, "norm_bwd_ring"),
             (Workload(dims=dict(rows=4096, hidden=4096), dtype="bfloat16"), 1, "norm_bwd_ring"))
    for w, route, kernel in cases:
        print(f"\n[gpu-parity] dispatch {name} {w.dims} {w.dtype}", flush=True)
        rep = verify(op, pair, device="cuda", workloads=(w,))
        assert rep.ok, "\n".join(rep.failures())
        inp = make_case_inputs(op, w, "cuda")
        args = [inp.get(a.name, getattr(a, "default", None)) for a in op.args]
        _, saved = fwd(*args)
        assert saved[0] == route and isinstance(saved[0], int)
        assert _first_bwd_kernel(bwd, inp["dy"], saved, eps=inp["eps"]) == kernel


@pytest.mark.parametrize("name", ["rmsnorm", "layernorm"])
def test_small_norm_program_gate_and_repeatability(name):
    """The small-shape program alone: every declared correctness workload (ragged
    widths, single rows, fp32/fp16/bf16), 512 rows (the most its one-launch backward
    takes) and the 1024-row sweep size (the ring) pass the gate; the one-launch
    backward is bitwise repeatable (fixed-order column sums, no atomics)."""
    import importlib

    from evograd_amd import SMALL_PROGRAMS
    from evograd_amd.opdecl import Workload

    op = decls.get_op(name)
    mod = importlib.import_module(SMALL_PROGRAMS[name])
    ws = list(op.correctness) + [Workload(dims=dict(rows=1024, hidden=4096), dtype="bfloat16"),
                                 Workload(dims=dict(rows=512, hidden=4096), dtype="bfloat16")]
    print(f"\n[gpu-parity] small {name} x{len(ws)}", flush=True)
    rep = verify(op, mod, device="cuda", workloads=tuple(ws))
    assert rep.ok, "\n".join(rep.failures())
    inp = make_case_inputs(op, ws[-1], "cuda")
    args = [inp.get(a.name, getattr(a, "default", None)) for a in op.args]
    _, saved = getattr(mod, op.forward_fn_name)(*args)
    bwd = getattr(mod, op.backward_fn_name)
    a = bwd(inp["dy"], saved, eps=inp["eps"])
    b = bwd(inp["dy"], saved, eps=inp["eps"])
    torch.cuda.synchronize()
    assert all(torch.equal(p, q) for p, q in zip(a, b))
