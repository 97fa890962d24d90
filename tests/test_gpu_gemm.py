"""The MFMA product behind the fused linear cross entropy (eg_gemm) against a torch
fp32 reference: every operand layout (k-contiguous or k-major A and B), ragged M,
N and k-major K, padded strides, fp32 / bf16 / fp16 outputs, and the fp32 path.
Bound: the fp32 result within fp32 accumulation rounding of the exact product of
the (exactly representable) 16-bit inputs; a 16-bit result within one rounding."""

import ctypes
import sys

import pytest
import torch

from evograd_amd import _lib

pytestmark = pytest.mark.gpu

LAYOUTS = [(True, True), (True, False), (False, False), (False, True)]
SHAPES = [(256, 256, 64), (300, 200, 128), (8, 512, 64), (1000, 777, 320), (260, 300, 100),
          (513, 1031, 192)]


def _r8(v):
    return (v + 7) // 8 * 8


def _operands(M, N, K, akc, bkc, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    A = torch.randn(M, K, device="cuda", generator=g).to(dtype)
    B = torch.randn(K, N, device="cuda", generator=g).to(dtype)
    if akc:
        lda = _r8(K)
        a = torch.zeros(M, lda, device="cuda", dtype=dtype)
        a[:, :K] = A
    else:
        lda = _r8(M)
        a = torch.zeros(K, lda, device="cuda", dtype=dtype)
        a[:, :M] = A.t()
    if bkc:
        ldb = _r8(K)
        b = torch.zeros(N, ldb, device="cuda", dtype=dtype)
        b[:, :K] = B.t()
    else:
        ldb = _r8(N)
        b = torch.zeros(K, ldb, device="cuda", dtype=dtype)
        b[:, :N] = B
    return A, B, a, b, lda, ldb


def _run(a, b, M, N, K, lda, ldb, akc, bkc, dtype, cdt):
    ldc = N + 3 if cdt == torch.float32 else _r8(N)
    c = torch.full((M, ldc), float("nan"), device="cuda", dtype=cdt)
    _lib.call("eg_gemm", a.data_ptr(), b.data_ptr(), c.data_ptr(), None, M, N, K, lda, ldb,
              ldc, 0, int(akc), int(bkc), _lib.dtype_tag(dtype), _lib.dtype_tag(cdt), None, 0,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return c


def _cases():
    for M, N, K in SHAPES:
        for akc, bkc in LAYOUTS:
            if (akc or bkc) and K % 64:
                continue
            yield pytest.param(M, N, K, akc, bkc, id=f"{M}x{N}x{K}-a{'k' if akc else 'm'}-b{'k' if bkc else 'n'}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K,akc,bkc", list(_cases()))
def test_gemm_16bit_operands_fp32_out(M, N, K, akc, bkc, dtype):
    print(f"\n[gpu-gemm] {dtype} {M}x{N}x{K} akc={akc} bkc={bkc}", flush=True)
    sys.stdout.flush()
    A, B, a, b, lda, ldb = _operands(M, N, K, akc, bkc, dtype, M + 7 * N + K)
    c = _run(a, b, M, N, K, lda, ldb, akc, bkc, dtype, torch.float32)
    ref = A.double() @ B.double()
    err = (c[:, :N].double() - ref).abs().max().item()
    # fp32 accumulation of K products of magnitude ~1: a few ulps of sqrt(K)
    assert err <= 4e-6 * K, err
    assert torch.isnan(c[:, N:]).all()  # columns past N untouched


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("akc,bkc", LAYOUTS)
def test_gemm_16bit_out_is_one_rounding(dtype, akc, bkc):
    M, N, K = 384, 320, 256
    A, B, a, b, lda, ldb = _operands(M, N, K, akc, bkc, dtype, 11)
    c = _run(a, b, M, N, K, lda, ldb, akc, bkc, dtype, dtype)
    ref = (A.double() @ B.double())
    rel = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    err = (c[:, :N].double() - ref).abs()
    assert (err <= rel * ref.abs() + 1e-5 * K).all(), err.max().item()


def test_gemm_fp32_path_and_zero_rows_past_the_operand():
    M, N, K = 130, 70, 45
    A, B, a, b, lda, ldb = _operands(M, N, K, False, False, torch.float32, 5)
    c = _run(a, b, M, N, K, lda, ldb, False, False, torch.float32, torch.float32)
    assert torch.allclose(c[:, :N].double(), A.double() @ B.double(), atol=1e-4, rtol=1e-5)
    A, B, a, b, lda, ldb = _operands(M, N, K, True, True, torch.float32, 6)
    c = _run(a, b, M, N, K, lda, ldb, True, True, torch.float32, torch.float32)
    assert torch.allclose(c[:, :N].double(), A.double() @ B.double(), atol=1e-4, rtol=1e-5)


def test_gemm_refuses_unsupported_shapes_on_the_host():
    x = torch.zeros(64, 64, device="cuda", dtype=torch.bfloat16)
    c = torch.zeros(64, 64, device="cuda")
    with pytest.raises(RuntimeError, match="K % 64"):
        _lib.call("eg_gemm", x.data_ptr(), x.data_ptr(), c.data_ptr(), None, 64, 64, 40, 64, 64,
                  64, 0, 1, 1, _lib.EG_BF16, _lib.EG_F32, None, 0,
                  torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("cdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("akc,bkc", [(True, True), (False, False), (True, False)])
@pytest.mark.parametrize("inplace", [False, True])
def test_gemm_residual_epilogue(cdt, akc, bkc, inplace):
    """c = r + a b with r added in fp32 before the one rounding of c; r == c
    accumulates in place (the fused linear cross entropy's dweight over row chunks,
    the decoder layer's residual adds)."""
    M, N, K = 300, 520, 128
    print(f"\n[gpu-gemm] residual {cdt} akc={akc} bkc={bkc} inplace={inplace}", flush=True)
    A, B, a, b, lda, ldb = _operands(M, N, K, akc, bkc, torch.bfloat16, 21)
    ldc = _r8(N) + 8
    g = torch.Generator(device="cuda").manual_seed(3)
    r = (torch.randn(M, ldc, device="cuda", generator=g) * 4).to(cdt)
    r0 = r.clone()
    if inplace:
        c, ldr = r, ldc
    else:
        c, ldr = torch.full((M, ldc), float("nan"), device="cuda", dtype=cdt), ldc
    _lib.call("eg_gemm", a.data_ptr(), b.data_ptr(), c.data_ptr(), r.data_ptr(), M, N, K, lda,
              ldb, ldc, ldr, int(akc), int(bkc), _lib.EG_BF16, _lib.dtype_tag(cdt), None, 0,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = r0[:, :N].double() + A.double() @ B.double()
    err = (c[:, :N].double() - ref).abs()
    if cdt == torch.float32:
        assert err.max().item() <= 4e-6 * K + 1e-6 * ref.abs().max().item()
    else:
        assert (err <= 2.0 ** -8 * ref.abs() + 1e-5 * K).all(), err.max().item()
    # columns past N: untouched (the residual's own values when in place)
    if inplace:
        assert torch.equal(c[:, N:], r0[:, N:])
    else:
        assert torch.isnan(c[:, N:]).all()
        assert torch.equal(r, r0)


def test_gemm_residual_fp32_path():
    M, N, K = 70, 90, 33
    A, B, a, b, lda, ldb = _operands(M, N, K, True, False, torch.float32, 8)
    r = torch.randn(M, N, device="cuda")
    c = torch.empty(M, N, device="cuda")
    _lib.call("eg_gemm", a.data_ptr(), b.data_ptr(), c.data_ptr(), r.data_ptr(), M, N, K, lda,
              ldb, N, N, 1, 0, _lib.EG_F32, _lib.EG_F32, None, 0,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.allclose(c.double(), r.double() + A.double() @ B.double(), atol=1e-4, rtol=1e-5)


@pytest.mark.parametrize("cdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K,akc,bkc", [(1024, 1024, 4096, True, True),
                                           (300, 700, 2048, True, False),
                                           (512, 256, 1000, False, False),
                                           (1024, 4096, 14336, True, True),
                                           # split tails: 272 tiles (the last 16 in 2 parts)
                                           (4300, 4000, 704, True, True),
                                           (4300, 4000, 704, True, False),
                                           (4300, 4000, 704, False, False),
                                           (4300, 4000, 704, False, True),
                                           # 896 tiles: the last 128 in 2 parts
                                           (4096, 14336, 1024, True, True)])
def test_gemm_split_k_matches_unsplit_and_is_repeatable(cdt, M, N, K, akc, bkc):
    """Few output tiles (split k) or a last wave of tiles at most half full (split
    tail), and a workspace: k parts into fp32 partials summed in a fixed order, the
    residual added and c rounded once. Against the unsplit product: the same sum in
    another order (fp32), and bitwise equal run to run."""
    print(f"\n[gpu-gemm] split-K {M}x{N}x{K} {cdt}", flush=True)
    need = _lib.query("eg_gemm_workspace_bytes", M, N, K, _lib.EG_BF16)
    assert need > 0
    A, B, a, b, lda, ldb = _operands(M, N, K, akc, bkc, torch.bfloat16, M + N + K)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    r = torch.randn(M, N, device="cuda").to(cdt)
    st = torch.cuda.current_stream().cuda_stream
    outs = []
    for work, nbytes in ((ws, need), (ws, need), (None, 0)):
        c = torch.full((M, N), float("nan"), device="cuda", dtype=cdt)
        _lib.call("eg_gemm", a.data_ptr(), b.data_ptr(), c.data_ptr(), r.data_ptr(), M, N, K,
                  lda, ldb, N, N, int(akc), int(bkc), _lib.EG_BF16, _lib.dtype_tag(cdt),
                  None if work is None else work.data_ptr(), nbytes, st)
        outs.append(c)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    ref = r.double() + A.double() @ B.double()
    for c in (outs[0], outs[2]):
        err = (c.double() - ref).abs()
        if cdt == torch.float32:
            assert err.max().item() <= 4e-6 * K, err.max().item()
        else:
            assert (err <= 2.0 ** -8 * ref.abs() + 4e-6 * K).all(), err.max().item()
    # a workspace one byte short runs unsplit (the same result as no workspace)
    c = torch.empty((M, N), device="cuda", dtype=cdt)
    _lib.call("eg_gemm", a.data_ptr(), b.data_ptr(), c.data_ptr(), r.data_ptr(), M, N, K, lda,
              ldb, N, N, int(akc), int(bkc), _lib.EG_BF16, _lib.dtype_tag(cdt), ws.data_ptr(),
              need - 1, st)
    torch.cuda.synchronize()
    assert torch.equal(c, outs[2])


# ------------------------------------------------------------- segmented operands
def _pieces(stored, along_rows, sizes, ld):
    """Split a stored [rows][cols] matrix into separate buffers of row stride ld,
    along its rows or its columns."""
    out, at = [], 0
    for n in sizes:
        part = stored[at:at + n] if along_rows else stored[:, at:at + n]
        buf = torch.zeros(part.shape[0], ld, device="cuda", dtype=stored.dtype)
        buf[:, :part.shape[1]] = part
        out.append(buf)
        at += n
    return out


SEG_CASES = [
    # dim, sizes, (M, N, K) with the segmented extent from sizes
    (1, [256, 512, 100], (None, 300, 384)),
    (2, [256, 256, 300], (300, None, 384)),
    (2, [256, 256, 300], (300, None, 2048)),          # split k, C in segments
    (2, [2048, 2048], (4352, None, 512)),             # split tail (272 tiles), C in segments
    (3, [128, 64, 192], (300, 400, None)),
    (3, [4096, 1024, 1024], (256, 512, None)),        # the decoder layer's q/k/v gradient
]


def _seg_cases():
    for dim, sizes, mnk in SEG_CASES:
        for akc, bkc in LAYOUTS:
            yield pytest.param(dim, sizes, mnk, akc, bkc,
                               id=f"d{dim}-{'-'.join(map(str, sizes))}-{mnk}-a{int(akc)}b{int(bkc)}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim,sizes,mnk,akc,bkc", list(_seg_cases()))
def test_gemm_segmented_is_the_concatenated_product_bitwise(dim, sizes, mnk, akc, bkc, dtype):
    """eg_gemm_segmented on operands cut into separate buffers along M, N or K gives
    the bits eg_gemm gives on the concatenated operands (same tiles, same k order,
    same split plan), for every layout; C in segments along M or N."""
    M, N, K = (sum(sizes) if v is None else v for v in mnk)
    print(f"\n[gpu-gemm] segmented {dtype} dim={dim} sizes={sizes} {M}x{N}x{K} a{int(akc)} b{int(bkc)}",
          flush=True)
    A, B, a, b, lda, ldb = _operands(M, N, K, akc, bkc, dtype, M * 3 + N + K + dim)
    st = torch.cuda.current_stream().cuda_stream
    tg = _lib.dtype_tag(dtype)
    need = _lib.query("eg_gemm_workspace_bytes", M, N, K, tg)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    ldc = _r8(N)
    want = torch.full((M, ldc), float("nan"), device="cuda", dtype=dtype)
    _lib.call("eg_gemm", a.data_ptr(), b.data_ptr(), want.data_ptr(), None, M, N, K, lda, ldb,
              ldc, 0, int(akc), int(bkc), tg, tg, ws.data_ptr(), need, st)
    # the operands the dimension indexes, cut into segments sharing one row stride
    a_segs = b_segs = c_segs = None
    seg_ld = _r8(max(sizes))
    if dim in (1, 3):  # A: rows m (k-contiguous) / columns m (k-major), or k
        a_rows = (dim == 1) == akc
        a_segs = _pieces(a[:, :(K if akc else M)], a_rows, sizes, lda if a_rows else seg_ld)
        seg_lda = lda if a_rows else seg_ld
    else:
        seg_lda = lda
    if dim in (2, 3):  # B: rows n (k-contiguous) / columns n, or k
        b_rows = (dim == 2) == bkc
        b_segs = _pieces(b[:, :(K if bkc else N)], b_rows, sizes, ldb if b_rows else seg_ld)
        seg_ldb = ldb if b_rows else seg_ld
    else:
        seg_ldb = ldb
    seg_ldc = ldc
    if dim in (1, 2):
        seg_ldc = ldc if dim == 1 else seg_ld
        c_segs = [torch.full((n if dim == 1 else M, seg_ldc), float("nan"), device="cuda",
                             dtype=dtype) for n in sizes]
    arr = lambda ts: (ctypes.c_void_p * len(sizes))(*[t.data_ptr() for t in ts]) if ts else None
    c = None if c_segs else torch.full((M, ldc), float("nan"), device="cuda", dtype=dtype)
    _lib.call("eg_gemm_segmented", None if a_segs else a.data_ptr(),
              None if b_segs else b.data_ptr(), None if c_segs else c.data_ptr(), M, N, K,
              seg_lda, seg_ldb, seg_ldc, int(akc), int(bkc), dim, len(sizes),
              (ctypes.c_int64 * len(sizes))(*sizes), arr(a_segs), arr(b_segs), arr(c_segs),
              tg, tg, ws.data_ptr(), need, st)
    if c_segs:
        got = torch.cat([t[:, :(N if dim == 1 else n)] for t, n in zip(c_segs, sizes)],
                        dim=0 if dim == 1 else 1)
    else:
        got = c[:, :N]
    torch.cuda.synchronize()
    assert torch.equal(got, want[:, :N])
    ref = A.double() @ B.double()
    ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    assert ((got.double() - ref).abs() <= ulp * ref.abs() + 4e-6 * K).all()

