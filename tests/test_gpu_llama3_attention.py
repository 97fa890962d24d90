"""Parity of the RoPE(q, k) -> grouped causal attention pair (llama3_attention).

The gate: the oracle restates the attention half of
src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:93-107 in fp32 and
differentiates it with torch.autograd.grad; bf16/fp16 tolerance 2e-2 / 1e-2 on o,
dq, dk, dv. Beyond it: the pair agrees with the two separate pairs it fuses (RoPE,
then GQA attention), its backward is bitwise repeatable, and it saves no rotated
copy of q or k.
"""

import sys

import pytest
import torch

from evograd_amd import decls, pair_module
from evograd_amd.harness import saved_state_report
from evograd_amd.inputs import make_case_inputs
from evograd_amd.opdecl import Workload
from oracle.verify import verify

pytestmark = pytest.mark.gpu
OP = decls.LLAMA3_ATTENTION


def _note(*parts):
    print("\n[gpu-llama3-attn]", *parts, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("w", OP.correctness, ids=lambda w: w.key())
def test_llama3_attention_correctness_workloads(w):
    _note(w.dims, w.dtype)
    rep = verify(OP, pair_module("llama3_attention"), device="cuda", workloads=(w,))
    torch.cuda.synchronize()
    assert rep.ok, "\n".join(rep.failures())


def test_llama3_attention_matches_rope_then_gqa():
    """o and the gradients against RoPE (the rope pair on q and k) followed by the
    GQA pair on the rotated tensors, the backward chained through both."""
    w = Workload(dims=dict(B=2, H=8, KVH=2, S=300, D=128), dtype="bfloat16")
    _note("vs rope + gqa", w.dims)
    inp = make_case_inputs(OP, w, "cuda")
    mod, rope, gqa = (pair_module(n) for n in ("llama3_attention", "rope", "causal_attention_gqa"))
    o, saved = mod.llama3_attention_forward_with_saved(inp["q"], inp["k"], inp["v"], inp["cos"],
                                                       inp["sin"])
    (qr, kr), rsaved = rope.rope_qk_forward_with_saved(inp["q"], inp["k"], inp["cos"], inp["sin"])
    o2, gsaved = gqa.causal_attention_gqa_forward_with_saved(qr, kr, inp["v"])
    assert torch.allclose(o.float(), o2.float(), atol=1e-2, rtol=1e-2)
    dq, dk, dv = mod.llama3_attention_backward_from_saved(inp["do"], saved)
    dqr, dkr, dv2 = gqa.causal_attention_gqa_backward_from_saved(inp["do"], gsaved)
    dq2, dk2 = rope.rope_qk_backward_from_saved((dqr, dkr), rsaved)
    for a, b in ((dq, dq2), (dk, dk2), (dv, dv2)):
        assert a.shape == b.shape and a.dtype == b.dtype
        assert torch.allclose(a.float(), b.float(), atol=3e-2, rtol=2e-2), (a.float() - b.float()).abs().max()


def test_llama3_attention_backward_is_bitwise_deterministic_and_saves_no_rotated_copy():
    w = Workload(dims=dict(B=1, H=32, KVH=8, S=1024, D=128), dtype="bfloat16")
    _note("determinism", w.dims)
    inp = make_case_inputs(OP, w, "cuda")
    mod = pair_module("llama3_attention")
    o, saved = mod.llama3_attention_forward_with_saved(inp["q"], inp["k"], inp["v"], inp["cos"],
                                                       inp["sin"])
    a = mod.llama3_attention_backward_from_saved(inp["do"], saved)
    b = mod.llama3_attention_backward_from_saved(inp["do"], saved)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    rep = saved_state_report(saved, {n: inp[n] for n in ("q", "k", "v", "cos", "sin")})
    # new storage: o and the fp32 logsumexp only (the fp32 tables are the caller's)
    assert rep["new_storage_bytes"] == o.numel() * o.element_size() + 1 * 32 * 1024 * 4
    assert saved[0] is inp["q"] and saved[1] is inp["k"]


def test_llama3_attention_llama3_8b_config():
    w = OP.benchmark[0]
    _note("llama3_8b", w.dims)
    rep = verify(OP, pair_module("llama3_attention"), device="cuda", workloads=(w,))
    torch.cuda.empty_cache()
    assert rep.ok, "\n".join(rep.failures())


def test_llama3_attention_tables_in_the_tensors_dtype():
    """Tables in x's dtype (as the reference decoder layer passes them,
    llama3_decoder_layer/__init__.py:122-123): the pair rotates with fp32 copies of
    them, so o and the gradients equal those of the same tables given in fp32, bit
    for bit, and the saved state holds the two fp32 copies as new storage."""
    w = Workload(dims=dict(B=1, H=8, KVH=2, S=200, D=128), dtype="bfloat16")
    _note("bf16 tables", w.dims)
    inp = make_case_inputs(OP, w, "cuda")
    mod = pair_module("llama3_attention")
    cos16, sin16 = inp["cos"].bfloat16(), inp["sin"].bfloat16()
    args = (inp["q"], inp["k"], inp["v"])
    o16, s16 = mod.llama3_attention_forward_with_saved(*args, cos16, sin16)
    o32, s32 = mod.llama3_attention_forward_with_saved(*args, cos16.float(), sin16.float())
    g16 = mod.llama3_attention_backward_from_saved(inp["do"], s16)
    g32 = mod.llama3_attention_backward_from_saved(inp["do"], s32)
    torch.cuda.synchronize()
    assert torch.equal(o16, o32)
    assert all(torch.equal(a, b) for a, b in zip(g16, g32))
    rep = saved_state_report(s16, {"q": inp["q"], "k": inp["k"], "v": inp["v"], "cos": cos16,
                                   "sin": sin16})
    S, D = w.dims["S"], w.dims["D"]
    assert rep["new_storage_bytes"] == (o16.numel() * o16.element_size() + 8 * S * 4
                                        + 2 * S * D * 4)
