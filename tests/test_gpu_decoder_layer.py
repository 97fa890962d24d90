"""The Llama-3 decoder layer pair (GPU) against the autograd oracle, plus the layout
and elementwise kernels it is built from.

The gate is the reference's own for this operator
(src/evograd/ops/level3/llama3_decoder_layer/__init__.py:55-65, :220-233): fp32 at
atol = rtol = 1e-4 and bf16 at atol 5e-2 / rtol 2e-2 against an fp32 reference
(atol x1.5 for dk_weight, dv_weight and ddown_weight), on the reference's four
small workloads (head_dim 32 and 16: the generic attention kernels) and on its
timed grid, B=1 and T in {1024, 2048, 4096} at Llama-3-8B widths (MFMA attention
and products)."""

import sys

import pytest
import torch

from evograd_amd import _lib, decls, pair_module
from evograd_amd.inputs import make_case_inputs, rope_tables
from oracle import forward_refs as fr
from oracle.verify import verify

pytestmark = pytest.mark.gpu

OP = decls.LLAMA3_DECODER_LAYER


def _note(*what):
    print(f"\n[gpu-layer] {' '.join(str(w) for w in what)}", flush=True)
    sys.stdout.flush()


def _cases(ws):
    for w in ws:
        yield pytest.param(w, id=f"{w.dtype}-{w.label or w.key()}")


@pytest.mark.parametrize("w", list(_cases(OP.correctness)))
def test_layer_correctness_workloads(w):
    _note(w.dims, w.dtype)
    rep = verify(OP, pair_module(OP.name), device="cuda", workloads=(w,))
    torch.cuda.synchronize()
    assert rep.ok, "\n".join(rep.failures())


@pytest.mark.parametrize("w", list(_cases(OP.benchmark)))
def test_layer_llama3_8b_widths(w):
    _note(w.dims, w.dtype)
    rep = verify(OP, pair_module(OP.name), device="cuda", workloads=(w,))
    torch.cuda.synchronize()
    assert rep.ok, "\n".join(rep.failures())
    torch.cuda.empty_cache()


def test_layer_fused_projections_at_whole_tile_widths():
    """Widths in whole 256-wide tiles (16-bit): q/k/v and gate/up run as single
    products over segmented weights (eg_gemm_segmented), and their gradients too;
    held to the same gate as every other workload (the small workloads above take
    the separate products)."""
    from evograd_amd.opdecl import Workload

    w = Workload(dims=dict(B=1, T=256, hidden=512, head_dim=64, q_out=512, kv_out=256,
                           intermediate=768), dtype="bfloat16")
    _note("fused", w.dims)
    rep = verify(OP, pair_module(OP.name), device="cuda", workloads=(w,))
    torch.cuda.synchronize()
    assert rep.ok, "\n".join(rep.failures())


def _run(inp, mod):
    args = [inp.get(a.name, getattr(a, "default", None)) for a in OP.args]
    out, saved = mod.llama3_decoder_layer_forward_with_saved(*args)
    grads = mod.llama3_decoder_layer_backward_from_saved(inp["dout"], saved, eps=inp["eps"])
    return out, saved, grads


def test_layer_is_bitwise_repeatable_and_saves_what_it_declares():
    """No atomics anywhere in the layer: two runs give identical bits. The saved state
    holds the inputs by reference plus o, lse, x1 and the two rstd vectors."""
    w = OP.benchmark[0]
    _note("repeat", w.dims)
    mod = pair_module(OP.name)
    inp = make_case_inputs(OP, w, "cuda")
    out1, saved, g1 = _run(inp, mod)
    out2, _, g2 = _run(inp, mod)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)
    args = {a.name: inp[a.name] for a in OP.args if torch.is_tensor(inp.get(a.name))}
    ids = {t.data_ptr() for t in args.values()}
    new = [t for t in saved if torch.is_tensor(t) and t.data_ptr() not in ids]
    d = w.dims
    M = d["B"] * d["T"]
    want = sorted([M * 4, M * 4, M * d["q_out"] * 2, M * d["hidden"] * 2,
                   d["B"] * (d["q_out"] // d["head_dim"]) * d["T"] * 4])
    assert sorted(t.numel() * t.element_size() for t in new) == want


# ----------------------------------------------------------- helper kernels
# one unit in the last place, relative (fp32: a few, for the fp32 evaluation itself)
_ULP = {torch.float32: 2.0 ** -20, torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}


def _stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D,heads,ld_pad", [(128, 4, 0), (32, 3, 8), (16, 2, 0), (6, 2, 2)])
@pytest.mark.parametrize("table_dtype", [torch.float32, "same"])
def test_split_merge_heads_with_rope(dtype, D, heads, ld_pad, table_dtype):
    _note("heads", dtype, D, heads, ld_pad, table_dtype)
    B, T = 2, 37
    ld = heads * D + ld_pad
    tdt = dtype if table_dtype == "same" else table_dtype
    g = torch.Generator(device="cuda").manual_seed(D + heads)
    src = torch.randn(B * T, ld, device="cuda", generator=g).to(dtype)
    cos, sin = rope_tables(T, D, 10000.0, tdt, "cuda")
    tg, ttg = _lib.dtype_tag(dtype), _lib.dtype_tag(tdt)
    view = src[:, :heads * D].reshape(B, T, heads, D).transpose(1, 2)
    for rope in (0, 1):
        dst = torch.empty(B, heads, T, D, device="cuda", dtype=dtype)
        _lib.call("eg_split_heads", src.data_ptr(), dst.data_ptr(), cos.data_ptr(),
                  sin.data_ptr(), B, T, heads, D, ld, rope, ttg, tg, _stream())
        torch.cuda.synchronize()
        if rope:
            # fp32 arithmetic, one rounding: within one unit of the last place of the
            # torch evaluation (which rounds its products separately)
            want = fr.rope_forward_ref(view.contiguous(), cos, sin)
            assert torch.allclose(dst.double(), want.double(), rtol=_ULP[dtype], atol=1e-6)
        else:
            assert torch.equal(dst, view.contiguous())
    # merge back, plain and with the rotation's transpose (the RoPE backward)
    hm = torch.randn(B, heads, T, D, device="cuda", generator=g).to(dtype)
    for rope in (0, 2):
        out = torch.full((B * T, ld), 7.0, device="cuda", dtype=dtype)
        _lib.call("eg_merge_heads", hm.data_ptr(), out.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                  B, T, heads, D, ld, rope, ttg, tg, _stream())
        torch.cuda.synchronize()
        want = (fr.rope_forward_ref(hm, cos, -sin) if rope else hm)
        want = want.transpose(1, 2).reshape(B * T, heads * D)
        if rope:
            assert torch.allclose(out[:, :heads * D].double(), want.double(), rtol=_ULP[dtype],
                                  atol=1e-6)
        else:
            assert torch.equal(out[:, :heads * D], want)
        assert (out[:, heads * D:] == 7.0).all()  # padding columns untouched


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,hq,hkv,ld_pad", [(128, 4, 2, 0), (64, 4, 4, 0), (32, 6, 3, 8),
                                              (6, 2, 1, 2)])
@pytest.mark.parametrize("table_dtype", [torch.float32, "same"])
def test_qkv_heads_equal_three_separate_layout_changes(dtype, D, hq, hkv, ld_pad, table_dtype):
    """eg_split_qkv_heads / eg_merge_qkv_heads (q, k and v of one fused projection in
    one launch) give the bits of eg_split_heads / eg_merge_heads on the three column
    ranges: q and k rotated (or transpose-rotated), v copied, padding columns of the
    merged rows untouched."""
    _note("qkv heads", dtype, D, hq, hkv, ld_pad, table_dtype)
    B, T = 2, 37
    ld = (hq + 2 * hkv) * D + ld_pad
    tdt = dtype if table_dtype == "same" else table_dtype
    g = torch.Generator(device="cuda").manual_seed(3 * D + hq)
    src = torch.randn(B * T, ld, device="cuda", generator=g).to(dtype)
    cos, sin = rope_tables(T, D, 10000.0, tdt, "cuda")
    tg, ttg = _lib.dtype_tag(dtype), _lib.dtype_tag(tdt)
    cols = (0, hq * D, (hq + hkv) * D)  # first column of q, k, v in a row
    nh = (hq, hkv, hkv)

    def heads(n):
        return torch.empty(B, n, T, D, device="cuda", dtype=dtype)

    fused = [heads(n) for n in nh]
    _lib.call("eg_split_qkv_heads", src.data_ptr(), *(t.data_ptr() for t in fused),
              cos.data_ptr(), sin.data_ptr(), B, T, hq, hkv, D, ld, 1, ttg, tg, _stream())
    for j in range(3):
        one = heads(nh[j])
        _lib.call("eg_split_heads", src[:, cols[j]:].data_ptr(), one.data_ptr(), cos.data_ptr(),
                  sin.data_ptr(), B, T, nh[j], D, ld, 1 if j < 2 else 0, ttg, tg, _stream())
        torch.cuda.synchronize()
        assert torch.equal(fused[j], one), f"split of tensor {j}"
    grads = [torch.randn(B, n, T, D, device="cuda", generator=g).to(dtype) for n in nh]
    out = torch.full((B * T, ld), 7.0, device="cuda", dtype=dtype)
    _lib.call("eg_merge_qkv_heads", *(t.data_ptr() for t in grads), out.data_ptr(),
              cos.data_ptr(), sin.data_ptr(), B, T, hq, hkv, D, ld, 2, ttg, tg, _stream())
    want = torch.full((B * T, ld), 7.0, device="cuda", dtype=dtype)
    for j in range(3):
        _lib.call("eg_merge_heads", grads[j].data_ptr(), want[:, cols[j]:].data_ptr(),
                  cos.data_ptr(), sin.data_ptr(), B, T, nh[j], D, ld, 2 if j < 2 else 0, ttg, tg,
                  _stream())
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    assert (out[:, (hq + 2 * hkv) * D:] == 7.0).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [1, 1000, 4096 * 33])
def test_add_and_silu_mul(dtype, n):
    _note("add/silu_mul", dtype, n)
    g = torch.Generator(device="cuda").manual_seed(n)
    a = (torch.randn(n, device="cuda", generator=g) * 4).to(dtype)
    b = torch.randn(n, device="cuda", generator=g).to(dtype)
    c = torch.empty_like(a)
    _lib.call("eg_add", a.data_ptr(), b.data_ptr(), c.data_ptr(), n, _lib.dtype_tag(dtype),
              _stream())
    torch.cuda.synchronize()
    assert torch.equal(c, (a.float() + b.float()).to(dtype))
    _lib.call("eg_silu_mul", a.data_ptr(), b.data_ptr(), c.data_ptr(), n, _lib.dtype_tag(dtype),
              _stream())
    torch.cuda.synchronize()
    want = torch.nn.functional.silu(a.double()) * b.double()  # one rounding of this
    err = (c.double() - want).abs()
    # plus half the spacing of the dtype's subnormals (fp16 results below 2^-14)
    tiny = 2.0 ** -25 if dtype == torch.float16 else 1e-38
    assert (err <= _ULP[dtype] * want.abs() + tiny).all(), float(err.max())
