"""Parity of the causal-attention HIP pair (MFMA) with the autograd oracle.

The oracle is causal softmax(q k^T / sqrt(D)) v written out in fp32
(oracle/forward_refs.py) differentiated by torch.autograd.grad; the gate is the
declaration's bf16/fp16 tolerance (2e-2 / 1e-2, atol and rtol) on o, dq, dk, dv.
"""

import sys

import pytest
import torch

from evograd_amd import decls, pair_module
from evograd_amd.inputs import make_case_inputs
from evograd_amd.opdecl import Workload
from oracle.forward_refs import causal_attention_lse_ref
from oracle.verify import verify

pytestmark = pytest.mark.gpu
OP = decls.CAUSAL_ATTENTION


def _note(*parts):
    print("\n[gpu-attn]", *parts, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("w", OP.correctness, ids=lambda w: w.key())
def test_attention_correctness_workloads(w):
    _note(w.dims, w.dtype)
    rep = verify(OP, pair_module("causal_attention"), device="cuda", workloads=(w,))
    assert rep.ok, "\n".join(rep.failures())


def test_attention_lse_matches_logsumexp():
    w = Workload(dims=dict(B=2, H=3, S=300, D=128), dtype="bfloat16")
    _note("lse", w.dims)
    inp = make_case_inputs(OP, w, "cuda")
    mod = pair_module("causal_attention")
    _, saved = mod.causal_attention_forward_with_saved(inp["q"], inp["k"], inp["v"])
    lse = saved[-1]
    ref = causal_attention_lse_ref(inp["q"], inp["k"])
    assert lse.dtype == torch.float32 and lse.shape == ref.shape
    assert torch.allclose(lse, ref, atol=1e-3, rtol=1e-4), (lse - ref).abs().max()


def test_attention_single_token_returns_v():
    g = torch.Generator(device="cuda").manual_seed(5)
    q, k, v = (torch.randn(2, 4, 1, 64, device="cuda", generator=g).bfloat16() for _ in range(3))
    o, _ = pair_module("causal_attention").causal_attention_forward_with_saved(q, k, v)
    assert torch.equal(o, v)


def test_attention_backward_is_bitwise_deterministic():
    w = Workload(dims=dict(B=1, H=4, S=1024, D=128), dtype="bfloat16")
    _note("determinism", w.dims)
    inp = make_case_inputs(OP, w, "cuda")
    mod = pair_module("causal_attention")
    _, saved = mod.causal_attention_forward_with_saved(inp["q"], inp["k"], inp["v"])
    a = mod.causal_attention_backward_from_saved(inp["do"], saved)
    b = mod.causal_attention_backward_from_saved(inp["do"], saved)
    assert all(torch.equal(x, y) for x, y in zip(a, b))


def test_attention_baseline_config():
    w = OP.benchmark[0]
    _note("baseline", w.dims)
    rep = verify(OP, pair_module("causal_attention"), device="cuda", workloads=(w,))
    torch.cuda.empty_cache()
    assert rep.ok, "\n".join(rep.failures())


GQA = decls.CAUSAL_ATTENTION_GQA


@pytest.mark.parametrize("w", GQA.correctness, ids=lambda w: w.key())
def test_attention_gqa_correctness_workloads(w):
    _note("gqa", w.dims, w.dtype)
    rep = verify(GQA, pair_module("causal_attention_gqa"), device="cuda", workloads=(w,))
    assert rep.ok, "\n".join(rep.failures())


def test_attention_gqa_matches_mha_on_repeated_kv():
    """The GQA kernels read each kv head in place of a repeated copy: o, lse and dq
    are bitwise those of the MHA kernels on repeat_interleave'd k, v; dk, dv are the
    group sums of the MHA gradients (one rounding instead of one per head)."""
    w = Workload(dims=dict(B=2, H=8, KVH=2, S=300, D=128), dtype="bfloat16")
    _note("gqa vs mha", w.dims)
    inp = make_case_inputs(GQA, w, "cuda")
    mha, gqa = pair_module("causal_attention"), pair_module("causal_attention_gqa")
    kr, vr = (inp[n].repeat_interleave(4, dim=1).contiguous() for n in ("k", "v"))
    og, sg = gqa.causal_attention_gqa_forward_with_saved(inp["q"], inp["k"], inp["v"])
    om, sm = mha.causal_attention_forward_with_saved(inp["q"], kr, vr)
    assert torch.equal(og, om) and torch.equal(sg[-1], sm[-1])
    dqg, dkg, dvg = gqa.causal_attention_gqa_backward_from_saved(inp["do"], sg)
    dqm, dkm, dvm = mha.causal_attention_backward_from_saved(inp["do"], sm)
    assert torch.equal(dqg, dqm)
    for a, b in ((dkg, dkm), (dvg, dvm)):
        ref = b.float().view(2, 2, 4, 300, 128).sum(2)
        assert a.shape == (2, 2, 300, 128)
        assert torch.allclose(a.float(), ref, atol=3e-2, rtol=2e-2), (a.float() - ref).abs().max()


def test_attention_gqa_backward_is_bitwise_deterministic():
    w = Workload(dims=dict(B=1, H=32, KVH=8, S=1024, D=128), dtype="bfloat16")
    _note("gqa determinism", w.dims)
    inp = make_case_inputs(GQA, w, "cuda")
    mod = pair_module("causal_attention_gqa")
    _, saved = mod.causal_attention_gqa_forward_with_saved(inp["q"], inp["k"], inp["v"])
    a = mod.causal_attention_gqa_backward_from_saved(inp["do"], saved)
    b = mod.causal_attention_gqa_backward_from_saved(inp["do"], saved)
    assert all(torch.equal(x, y) for x, y in zip(a, b))


def test_attention_gqa_split_dkdv_walk():
    """Few (kv head, key block) pairs: the dK/dV walk is cut into parts summed in
    fp32 slabs (B=1, 8 kv heads, 8 key blocks: 8 parts), held to the oracle like
    every other workload, and repeatable bitwise."""
    w = Workload(dims=dict(B=1, H=32, KVH=8, S=1024, D=128), dtype="bfloat16")
    _note("gqa split walk", w.dims)
    rep = verify(GQA, pair_module("causal_attention_gqa"), device="cuda", workloads=(w,))
    assert rep.ok, "\n".join(rep.failures())


def test_attention_gqa_llama3_8b_config():
    w = GQA.benchmark[0]
    _note("gqa llama3_8b", w.dims)
    rep = verify(GQA, pair_module("causal_attention_gqa"), device="cuda", workloads=(w,))
    torch.cuda.empty_cache()
    assert rep.ok, "\n".join(rep.failures())
