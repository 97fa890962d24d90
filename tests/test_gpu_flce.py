"""Parity of the fused linear cross-entropy pair (this library's MFMA products and row kernels).

The declaration's cases run the reference's gate (oracle: fp32 logits, autograd).
Beyond it: the chunked result equals the single-chunk one and an fp64 evaluation
to within the roundings the pair performs (the unit gradient to the input dtype,
dx and dweight each rounded at the end of the forward and again after the dloss
scaling), the saved state holds nothing of size rows x vocab, and the benchmark
Llama-3-8B size passes the gate.
"""

import sys

import pytest
import torch

from evograd_amd import decls, pair_module
from evograd_amd.bind import bind
from evograd_amd.inputs import make_case_inputs
from evograd_amd.opdecl import Workload
from oracle.verify import verify

pytestmark = pytest.mark.gpu
OP = decls.FUSED_LINEAR_CROSS_ENTROPY


def _note(*parts):
    print("\n[gpu-flce]", *parts, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("w", OP.correctness, ids=lambda w: w.key())
def test_flce_correctness_workloads(w):
    _note(w.dims, w.dtype, w.extra)
    rep = verify(OP, pair_module("fused_linear_cross_entropy"), device="cuda", workloads=(w,))
    torch.cuda.synchronize()
    assert rep.ok, "\n".join(rep.failures())


def _ref64(inp):
    x = inp["x"].double().requires_grad_(True)
    wt = inp["weight"].double().requires_grad_(True)
    loss = torch.nn.functional.cross_entropy(x @ wt.t(), inp["target"], ignore_index=-100)
    gx, gw = torch.autograd.grad(loss, (x, wt), grad_outputs=inp["dloss"].double())
    return loss.detach(), gx, gw


def _close(a, ref, rel):
    err = (a.double() - ref).abs()
    bound = rel * ref.abs() + rel * ref.abs().mean()
    return float((err - bound).max()) <= 0, float(err.max())


@pytest.mark.parametrize("vocab", [4096, 8200])
def test_flce_chunked_equals_single_chunk_and_fp64(vocab):
    """Five chunks of 64 rows (the last one ragged) against one chunk and fp64: the
    per-row fix-up loop (4096 columns) and the flat fix-up pass over each chunk (8200
    columns, padded rows)."""
    mod = pair_module("fused_linear_cross_entropy")
    w = Workload(dims=dict(rows=300, hidden=256, vocab=vocab), dtype="bfloat16",
                 extra={"ignore_every": 7})
    _note("chunking", w.dims)
    inp = make_case_inputs(OP, w, "cuda")
    args = (inp["x"], inp["weight"], inp["target"])
    one_loss, one_saved = mod.fused_linear_cross_entropy_forward_with_saved(*args)
    one = mod.fused_linear_cross_entropy_backward_from_saved(inp["dloss"], one_saved)
    old = mod.CHUNK_ELEMS
    mod.CHUNK_ELEMS = 64 * vocab  # 64-row chunks: 5 chunks, the last one ragged
    try:
        assert mod.chunk_rows(300, vocab) == 64
        many_loss, many_saved = mod.fused_linear_cross_entropy_forward_with_saved(*args)
        many = mod.fused_linear_cross_entropy_backward_from_saved(inp["dloss"], many_saved)
    finally:
        mod.CHUNK_ELEMS = old
    torch.cuda.synchronize()
    ref_loss, ref_dx, ref_dw = _ref64(inp)
    for loss in (one_loss, many_loss):
        assert loss.dtype == torch.float32
        assert abs(float(loss) - float(ref_loss)) <= 1e-5 * abs(float(ref_loss))
    for dx, dw in (one, many):
        ok, e = _close(dx, ref_dx, 2.0 ** -6)
        assert ok, f"dx max err {e:.3g}"
        ok, e = _close(dw, ref_dw, 2.0 ** -6)
        assert ok, f"dweight max err {e:.3g}"
    # dx rows do not depend on the split; dweight takes one more rounding per chunk
    # (each chunk's product is added to the running sum in fp32, then rounded)
    assert torch.equal(one[0], many[0])
    ok, e = _close(many[1], one[1].double(), 2.0 ** -6)
    assert ok, f"chunked dweight differs from one chunk by {e:.3g}"
    # saved state: the two gradients and one count, nothing rows x vocab
    assert [tuple(t.shape) for t in many_saved] == [(300, 256), (vocab, 256), (1,)]


@pytest.mark.parametrize("dtype,hidden", [("bfloat16", 100), ("float16", 200)])
def test_flce_hidden_not_a_multiple_of_the_k_step(dtype, hidden):
    """16-bit inputs whose hidden size is not a multiple of 64 go through zero-padded
    copies; the padding adds nothing to the logits and is cut from dx."""
    mod = pair_module("fused_linear_cross_entropy")
    w = Workload(dims=dict(rows=77, hidden=hidden, vocab=1000), dtype=dtype,
                 extra={"ignore_every": 5})
    _note("odd hidden", w.dims, dtype)
    inp = make_case_inputs(OP, w, "cuda")
    loss, saved = mod.fused_linear_cross_entropy_forward_with_saved(
        inp["x"], inp["weight"], inp["target"])
    dx, dw = mod.fused_linear_cross_entropy_backward_from_saved(inp["dloss"], saved)
    torch.cuda.synchronize()
    assert dx.shape == inp["x"].shape and dw.shape == inp["weight"].shape
    ref_loss, ref_dx, ref_dw = _ref64(inp)
    assert abs(float(loss) - float(ref_loss)) <= 1e-5 * abs(float(ref_loss))
    # each entry within 2^-6 of the sum of the absolute terms of its dot product
    # (the unit gradient rounded to 16 bits, the results rounded twice more)
    x, wt, target = inp["x"].double(), inp["weight"].double(), inp["target"]
    dl = torch.softmax(x @ wt.t(), dim=1)
    keep = target != -100
    dl[keep, target[keep]] -= 1.0
    dl = dl * keep[:, None] * (float(inp["dloss"]) / float(keep.sum()))
    bound_x = 2.0 ** -6 * (dl.abs() @ wt.abs())
    bound_w = 2.0 ** -6 * (dl.abs().t() @ x.abs())
    assert bool(((dx.double() - ref_dx).abs() <= bound_x + 1e-12).all())
    assert bool(((dw.double() - ref_dw).abs() <= bound_w + 1e-12).all())


def test_flce_through_autograd_binding():
    mod = pair_module("fused_linear_cross_entropy")
    w = OP.correctness[1]
    _note("bind", w.dims, w.dtype)
    inp = make_case_inputs(OP, w, "cuda")
    x = inp["x"].detach().clone().requires_grad_(True)
    wt = inp["weight"].detach().clone().requires_grad_(True)
    loss = bind(OP, mod)(x, wt, inp["target"])
    loss.backward()
    _, saved = mod.fused_linear_cross_entropy_forward_with_saved(inp["x"], inp["weight"],
                                                                 inp["target"])
    gx, gw = mod.fused_linear_cross_entropy_backward_from_saved(
        torch.ones((), device="cuda", dtype=torch.float32), saved)
    assert torch.allclose(x.grad.float(), gx.float(), rtol=1e-2, atol=1e-6)
    assert torch.allclose(wt.grad.float(), gw.float(), rtol=1e-2, atol=1e-6)


def test_flce_llama_size_gate():
    w = OP.benchmark[0]
    _note("llama size", w.dims, w.dtype)
    rep = verify(OP, pair_module("fused_linear_cross_entropy"), device="cuda", workloads=(w,))
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    assert rep.ok, "\n".join(rep.failures())


@pytest.mark.parametrize("rows", [0, 24])
def test_flce_with_no_counted_row_has_zero_gradients(rows):
    """Every target ignored (or no rows at all): torch's loss is NaN (a mean over no
    rows) and its gradients are zero; the dloss / n scaling must not turn the zero
    unit gradients into NaN."""
    mod = pair_module("fused_linear_cross_entropy")
    _note("no counted row", rows)
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(rows, 64, device="cuda", dtype=torch.bfloat16, generator=g)
    wt = torch.randn(512, 64, device="cuda", dtype=torch.bfloat16, generator=g)
    target = torch.full((rows,), -100, device="cuda", dtype=torch.int64)
    loss, saved = mod.fused_linear_cross_entropy_forward_with_saved(x, wt, target)
    dx, dw = mod.fused_linear_cross_entropy_backward_from_saved(
        torch.ones((), device="cuda", dtype=torch.float32), saved)
    torch.cuda.synchronize()
    xr, wr = x.float().cpu().requires_grad_(True), wt.float().cpu().requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(xr @ wr.t(), target.cpu(), ignore_index=-100)
    rgx, rgw = torch.autograd.grad(ref, (xr, wr))
    assert torch.isnan(loss).item() and torch.isnan(ref).item()
    assert dx.shape == x.shape and dw.shape == wt.shape
    assert torch.equal(dx.float().cpu(), rgx) and torch.equal(dw.float().cpu(), rgw)
    assert not torch.isnan(dw).any().item() and int(torch.count_nonzero(dw)) == 0


def _torch_ref32(x, wt, target):
    xr = x.float().requires_grad_(True)
    wr = wt.float().requires_grad_(True)
    loss = torch.nn.functional.cross_entropy(xr @ wr.t(), target, ignore_index=-100)
    gx, gw = torch.autograd.grad(loss, (xr, wr))
    return loss.detach(), gx, gw


@pytest.mark.parametrize("vocab", [1000, 8200])
def test_flce_target_out_of_range_gives_nan_row(vocab):
    """A target outside [0, vocab) that is not ignore_index: the loss is NaN (torch
    raises there) and so is that row's gradient; the other rows of dx stay finite
    (the loop over each row, and the flat pass over wide rows)."""
    mod = pair_module("fused_linear_cross_entropy")
    _note("bad target", vocab)
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(40, 128, device="cuda", dtype=torch.bfloat16, generator=g)
    wt = torch.randn(vocab, 128, device="cuda", dtype=torch.bfloat16, generator=g)
    target = torch.randint(0, vocab, (40,), device="cuda", generator=g)
    target[7] = vocab
    loss, saved = mod.fused_linear_cross_entropy_forward_with_saved(x, wt, target)
    dx, _ = mod.fused_linear_cross_entropy_backward_from_saved(
        torch.ones((), device="cuda", dtype=torch.float32), saved)
    torch.cuda.synchronize()
    assert torch.isnan(loss).item()
    assert torch.isnan(dx[7].float()).all().item()
    others = torch.cat([dx[:7], dx[8:]]).float()
    assert torch.isfinite(others).all().item()


def test_flce_vocab_past_the_fused_limit_takes_the_fp32_path():
    """16-bit inputs whose rows hold more than 8192 softmax groups (vocab > 2^20)
    run the fp32-logits chunk path; both paths must agree with torch."""
    mod = pair_module("fused_linear_cross_entropy")
    vocab = (1 << 20) + 128
    _note("vocab", vocab)
    g = torch.Generator(device="cuda").manual_seed(12)
    x = torch.randn(4, 64, device="cuda", dtype=torch.bfloat16, generator=g)
    wt = (0.25 * torch.randn(vocab, 64, device="cuda", generator=g)).bfloat16()
    target = torch.tensor([3, vocab - 1, -100, 1 << 19], device="cuda")
    loss, saved = mod.fused_linear_cross_entropy_forward_with_saved(x, wt, target)
    dloss = torch.full((), 2.0, device="cuda", dtype=torch.float32)
    dx, dw = mod.fused_linear_cross_entropy_backward_from_saved(dloss, saved)
    ref_loss, rgx, rgw = _torch_ref32(x, wt, target)
    torch.cuda.synchronize()
    assert abs(float(loss) - float(ref_loss)) <= 1e-4 * abs(float(ref_loss))
    # The unit gradient is rounded to bf16 before the products and the results are
    # rounded twice more (before and after the dloss / n scaling): each entry is
    # held to 2^-6 of the sum of the absolute terms of its dot product, which
    # covers that rounding also where the terms cancel (most of the 2^20 columns).
    logits = x.float() @ wt.float().t()
    dl = torch.softmax(logits, dim=1)
    keep = target != -100
    dl[keep, target[keep]] -= 1.0
    dl = dl * keep[:, None] * (2.0 / float(keep.sum()))
    bound_x = 2.0 ** -6 * (dl.abs() @ wt.float().abs())
    bound_w = 2.0 ** -6 * (dl.abs().t() @ x.float().abs())
    assert bool(((dx.float() - 2.0 * rgx).abs() <= bound_x + 1e-12).all())
    assert bool(((dw.float() - 2.0 * rgw).abs() <= bound_w + 1e-12).all())
    del wt, dw, rgw, dl, bound_w, logits
    torch.cuda.empty_cache()


@pytest.mark.parametrize("vocab,dtype", [(8184, torch.bfloat16), (8192, torch.bfloat16),
                                         (8200, torch.bfloat16), (8200, torch.float16),
                                         (131080, torch.bfloat16)])
def test_flce_fixup_row_width_edges(vocab, dtype):
    """The fix-up takes rows of whole 8-column packs from 8192 columns on as one flat
    pass over the chunk (a workgroup's 1024 packs may span two rows) and loops over
    each narrower row: the last width of the loop, the first of the flat pass (rows
    of exactly one workgroup), one where workgroups span rows, and a wide padded one,
    with targets in the first and last columns, an ignored row and a target in the
    last 128-column group, agree with torch."""
    mod = pair_module("fused_linear_cross_entropy")
    _note("fix-up width", vocab, dtype)
    g = torch.Generator(device="cuda").manual_seed(13)
    x = torch.randn(6, 64, device="cuda", generator=g).to(dtype)
    wt = (0.25 * torch.randn(vocab, 64, device="cuda", generator=g)).to(dtype)
    target = torch.tensor([0, vocab - 1, -100, vocab - 100, vocab // 2, 12345 % vocab],
                          device="cuda")
    loss, saved = mod.fused_linear_cross_entropy_forward_with_saved(x, wt, target)
    dloss = torch.full((), 1.5, device="cuda", dtype=torch.float32)
    dx, dw = mod.fused_linear_cross_entropy_backward_from_saved(dloss, saved)
    ref_loss, rgx, rgw = _torch_ref32(x, wt, target)
    torch.cuda.synchronize()
    assert abs(float(loss) - float(ref_loss)) <= 1e-4 * abs(float(ref_loss))
    # each entry within 2^-6 of the sum of the absolute terms of its dot product (the
    # unit gradient rounded to 16 bits, the results rounded twice more)
    logits = x.float() @ wt.float().t()
    dl = torch.softmax(logits, dim=1)
    keep = target != -100
    dl[keep, target[keep]] -= 1.0
    scale = 1.5 / float(keep.sum())
    dl = dl * keep[:, None] * scale
    bound_x = 2.0 ** -6 * (dl.abs() @ wt.float().abs())
    bound_w = 2.0 ** -6 * (dl.abs().t() @ x.float().abs())
    if dtype == torch.float16:
        # fp16 keeps values below 2^-14 as subnormals, spaced 2^-24 apart: each rounding
        # of a tiny value errs by up to 2^-25 absolute, which no relative bound covers.
        # The exponential and the unit gradient are rounded once each before the
        # products, the products' unit results once, and the scaled results once more.
        def floor(other):  # other: the |operand| summed along the product's k
            return scale * (2.0 ** -24 * other + 2.0 ** -25) + 2.0 ** -25
        bound_x = bound_x + floor(wt.float().abs().sum(0))[None, :]
        bound_w = bound_w + floor(x.float().abs()[keep].sum(0))[None, :]
    assert bool(((dx.float() - 1.5 * rgx).abs() <= bound_x + 1e-12).all())
    assert bool(((dw.float() - 1.5 * rgw).abs() <= bound_w + 1e-12).all())
    assert torch.equal(dx[2], torch.zeros_like(dx[2]))  # the ignored row
