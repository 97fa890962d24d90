"""The sustained-rate MFMA probes behind bench.py's "sustained" figures
(eg_probe_mfma_bf16, eg_probe_mfma_mix): checksums against the closed form of the
sum of a matrix product's elements, sum(A B) = sum_k colsum(A)[k] rowsum(B)[k], and
rates below the published dense bf16 peak."""

import pytest
import torch

from evograd_amd import _lib

pytestmark = pytest.mark.gpu

PACKS = 2048          # 16-byte operand packs the kernel reads
THREADS = 256
PEAK_TFLOPS = 2516.6


def _expected_wave_sums(operands: torch.Tensor, iters: int) -> torch.Tensor:
    """Sum of the checksums of each of the 4 waves of a workgroup, in float64.

    Thread t holds ra[s] = packs[(8t + s) % 2048] and rb[s] = packs[(8t + 4 + s) %
    2048]; accumulator (i, j) takes, per substep s, v_mfma_f32_32x32x16_bf16 with
    first operand rb[(s + 3j) & 3] (lane l: row l % 32, k = 8 (l / 32) + e) and
    second operand ra[(s + i) & 3] (lane l: column l % 32, same k). The elements of
    a 32 x 32 x 16 product sum to sum_k (sum over the rows of the first operand at
    k) x (sum over the columns of the second at k)."""
    packs = operands.view(torch.int16).view(PACKS, 8).view(torch.bfloat16).double().cpu()
    t = torch.arange(THREADS)
    ra = torch.stack([packs[(8 * t + s) % PACKS] for s in range(4)], 1)      # [256, 4, 8]
    rb = torch.stack([packs[(8 * t + 4 + s) % PACKS] for s in range(4)], 1)
    out = torch.zeros(4, dtype=torch.float64)
    for w in range(4):
        lanes = slice(64 * w, 64 * w + 64)
        # [4 sets, 2 halves, 8] sums over the 32 lanes of each half
        ca = ra[lanes].view(2, 32, 4, 8).sum(1).permute(1, 0, 2)
        cb = rb[lanes].view(2, 32, 4, 8).sum(1).permute(1, 0, 2)
        total = 0.0
        for s in range(4):
            for i in range(4):
                for j in range(4):
                    total += float((cb[(s + 3 * j) & 3] * ca[(s + i) & 3]).sum())
        out[w] = iters * total
    return out


def _run(operands, iters, workgroups):
    out = torch.full((workgroups * THREADS,), float("nan"), device="cuda")
    _lib.call("eg_probe_mfma_bf16", operands.data_ptr(), out.data_ptr(), workgroups, iters,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out


def test_probe_checksums_match_the_closed_form():
    g = torch.Generator(device="cuda").manual_seed(3)
    operands = torch.randn(PACKS * 8, device="cuda", generator=g).to(torch.bfloat16)
    assert torch.equal(_run(operands, 0, 4), torch.zeros(4 * THREADS, device="cuda"))
    for iters in (1, 3):
        out = _run(operands, iters, 4).double().cpu().view(4, 4, 64).sum(-1)  # [wg, wave]
        want = _expected_wave_sums(operands, iters)
        scale = iters * 64 * 64.0  # 64 products per iteration, |colsum| ~ 32 per side
        for wg in range(4):
            torch.testing.assert_close(out[wg], want, rtol=0, atol=1e-4 * scale)


def test_probe_rate_is_below_the_published_peak():
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    g = torch.Generator(device="cuda").manual_seed(5)
    operands = torch.randn(PACKS * 8, device="cuda", generator=g).to(torch.bfloat16)
    iters = 2000
    _run(operands, iters // 10, cus)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = torch.empty(cus * THREADS, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    e0.record()
    _lib.call("eg_probe_mfma_bf16", operands.data_ptr(), out.data_ptr(), cus, iters, stream)
    e1.record()
    e1.synchronize()
    tflops = cus * 4 * iters * 64 * 32768 / (e0.elapsed_time(e1) * 1e-3) / 1e12
    assert torch.isfinite(out).all()
    assert 0.2 * PEAK_TFLOPS < tflops < 1.01 * PEAK_TFLOPS, tflops


def _expected_wave_sums_16(operands: torch.Tensor, iters: int) -> torch.Tensor:
    """eg_probe_mfma_mix kind 1: accumulator t takes, per substep s (0..7),
    v_mfma_f32_16x16x32_bf16 with first operand rb[(s + 3 (t / 4)) & 3] (lane l:
    row l % 16, k = 8 (l / 16) + e) and second operand ra[(s + t) & 3] (column
    l % 16, same k), so each product's elements sum to sum_k (sum over the 16 lanes
    of each quarter of the first) x (the same of the second)."""
    packs = operands.view(torch.int16).view(PACKS, 8).view(torch.bfloat16).double().cpu()
    t = torch.arange(THREADS)
    ra = torch.stack([packs[(8 * t + s) % PACKS] for s in range(4)], 1)      # [256, 4, 8]
    rb = torch.stack([packs[(8 * t + 4 + s) % PACKS] for s in range(4)], 1)
    out = torch.zeros(4, dtype=torch.float64)
    for w in range(4):
        lanes = slice(64 * w, 64 * w + 64)
        ca = ra[lanes].view(4, 16, 4, 8).sum(1).permute(1, 0, 2)   # [set, quarter, 8]
        cb = rb[lanes].view(4, 16, 4, 8).sum(1).permute(1, 0, 2)
        total = 0.0
        for s in range(8):
            for tt in range(16):
                total += float((cb[(s + 3 * (tt >> 2)) & 3] * ca[(s + tt) & 3]).sum())
        out[w] = iters * total
    return out


def _run_mix(kind, operands, iters, workgroups):
    out = torch.full((workgroups * THREADS,), float("nan"), device="cuda")
    _lib.call("eg_probe_mfma_mix", kind, operands.data_ptr(), out.data_ptr(), workgroups, iters,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out


def test_mix_probe_kind0_is_the_register_probe_and_kind1_matches_its_closed_form():
    g = torch.Generator(device="cuda").manual_seed(3)
    operands = torch.randn(PACKS * 8, device="cuda", generator=g).to(torch.bfloat16)
    assert torch.equal(_run_mix(0, operands, 2, 4), _run(operands, 2, 4))
    for iters in (1, 3):
        out = _run_mix(1, operands, iters, 4).double().cpu().view(4, 4, 64).sum(-1)
        want = _expected_wave_sums_16(operands, iters)
        scale = iters * 128 * 16 * 16.0
        for wg in range(4):
            torch.testing.assert_close(out[wg], want, rtol=0, atol=1e-4 * scale)


@pytest.mark.parametrize("kind", [1, 2, 3])
def test_mix_probe_rates_are_below_the_published_peak(kind):
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    g = torch.Generator(device="cuda").manual_seed(5)
    operands = torch.randn(PACKS * 8, device="cuda", generator=g).to(torch.bfloat16)
    iters, wgs = 1000, 2 * cus
    _run_mix(kind, operands, iters // 10, wgs)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = torch.empty(wgs * THREADS, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    e0.record()
    _lib.call("eg_probe_mfma_mix", kind, operands.data_ptr(), out.data_ptr(), wgs, iters, stream)
    e1.record()
    e1.synchronize()
    tflops = wgs * 4 * iters * 64 * 32768 / (e0.elapsed_time(e1) * 1e-3) / 1e12
    assert torch.isfinite(out).all()
    assert 0.2 * PEAK_TFLOPS < tflops < 1.01 * PEAK_TFLOPS, tflops
