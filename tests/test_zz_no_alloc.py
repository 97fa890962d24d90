"""eg_rmsnorm_bwd_noalloc (partial rows in the library's device-resident scratch
array) gives exactly eg_rmsnorm_bwd's results (same kernels, caller-provided
workspace), called through the C ABI: two calls in a row, the second smaller, so
the second reads a scratch array the first left full of its own partial rows."""

import pytest
import torch

from evograd_amd import _lib

pytestmark = pytest.mark.gpu


def _case(rows, hidden, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(rows, hidden, device="cuda", dtype=dtype, generator=g)
    dy = torch.randn(rows, hidden, device="cuda", dtype=dtype, generator=g)
    w = (1 + 0.1 * torch.randn(hidden, device="cuda", generator=g)).to(dtype)
    rstd = torch.rsqrt(x.float().pow(2).mean(-1) + 1e-6).contiguous()
    return x, dy, w, rstd


def _with_workspace(x, dy, w, rstd):
    rows, hidden = x.shape
    dx, dw = torch.empty_like(x), torch.empty_like(w)
    ws = torch.empty(max(1, _lib.query("eg_rmsnorm_workspace_bytes", rows, hidden)),
                     dtype=torch.uint8, device="cuda")
    _lib.call("eg_rmsnorm_bwd", dy.data_ptr(), x.data_ptr(), w.data_ptr(), rstd.data_ptr(),
              dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), rows, hidden,
              _lib.dtype_tag(x.dtype), _lib.stream_of(x))
    return dx, dw


def _without(x, dy, w, rstd, dx, dw):
    rows, hidden = x.shape
    _lib.call("eg_rmsnorm_bwd_noalloc", dy.data_ptr(), x.data_ptr(), w.data_ptr(),
              rstd.data_ptr(), dx.data_ptr(), dw.data_ptr(), rows, hidden,
              _lib.dtype_tag(x.dtype), _lib.stream_of(x))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_backward_equals_the_workspace_entry_point(dtype):
    cases = [(16384, 4096, 11), (300, 1000, 12)]  # second call smaller (ragged width)
    inputs = [_case(r, h, dtype, s) for r, h, s in cases]
    expected = [_with_workspace(*c) for c in inputs]
    torch.cuda.synchronize()
    outs = [(torch.full_like(c[0], float("nan")), torch.full_like(c[2], float("nan")))
            for c in inputs]
    for (r, h, _), c, o in zip(cases, inputs, outs):
        print(f"\n[gpu-noalloc] rmsnorm bwd rows={r} hidden={h} {dtype}", flush=True)
        _without(*c, *o)
        torch.cuda.synchronize()
    for (dx, dw), (ex, ew) in zip(outs, expected):
        assert torch.equal(dx, ex) and torch.equal(dw, ew)


def test_noalloc_backward_with_no_rows_zeroes_dweight():
    # (sizes beyond the scratch are refused on the host before any launch:
    # tests/test_capi.py checks that without a GPU)
    x, dy, w, rstd = _case(0, 256, torch.bfloat16, 4)
    dw = torch.full((256,), float("nan"), device="cuda", dtype=torch.bfloat16)
    _without(x, dy, w, rstd, torch.empty_like(x), dw)
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(dw)) == 0
