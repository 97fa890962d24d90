// Sustained bf16 MFMA rates of the device, as a measurement aid for the roofline
// figures: the published dense peak (2516.6 TFLOP/s) assumes the 2.4 GHz engine
// clock, which the device holds only while the matrix cores see low-toggle data;
// with random bf16 operands power management lowers the clock. The register probes
// keep every SIMD's matrix core busy from registers alone (no memory traffic inside
// the loop), on operands the caller fills with random bf16 values, so their rate is
// the ceiling a kernel's MFMA work can approach on this device: one for each of the
// two bf16 MFMA shapes (32 x 32 x 16 at one wave per SIMD, 16 x 16 x 32 at two).
// The LDS probes feed every 32 x 32 x 16 MFMA one LDS operand read of 1 KiB per
// wave, the operand traffic of the attention kernels, optionally with one
// exponential per MFMA: the ceiling of a kernel whose operands come through LDS at
// that rate.
#include "eg_common.hpp"

namespace eg {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kProbeThreads = 256;
constexpr int kProbeOperandPacks = 2048;  // 16-byte packs read from `operands` (32 KiB)

// One workgroup of 4 waves per CU, one wave per SIMD. Per iteration each wave
// issues 64 v_mfma_f32_32x32x16_bf16 into 16 independent accumulators, cycling
// through 4 operand sets per side so consecutive MFMAs see different data.
__global__ __launch_bounds__(kProbeThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void mfma_probe_kernel(const u32x4* __restrict__ operands, float* __restrict__ out, int iters) {
  u32x4 ra[4], rb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    ra[s] = operands[(threadIdx.x * 8 + s) % kProbeOperandPacks];
    rb[s] = operands[(threadIdx.x * 8 + 4 + s) % kProbeOperandPacks];
  }
  f32x16 acc[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) acc[t] = f32x16{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bf16x8 a, b;
          __builtin_memcpy(&a, &ra[(s + i) & 3], 16);
          __builtin_memcpy(&b, &rb[(s + 3 * j) & 3], 16);
          acc[i * 4 + j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, acc[i * 4 + j], 0, 0, 0);
        }
  }
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < 16; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) sum += acc[t][r];
  out[(size_t)blockIdx.x * kProbeThreads + threadIdx.x] = sum;
}

// The same work per wave and iteration (64 x 32768 FLOP) as 128 v_mfma_f32_16x16x32_bf16
// into 16 independent accumulators, two workgroups per CU (two waves per SIMD: the
// 16 x 16 x 32 form reaches its sustained rate only with a second wave to issue).
__global__ __launch_bounds__(kProbeThreads, 2) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mfma16_probe_kernel(const u32x4* __restrict__ operands, float* __restrict__ out, int iters) {
  u32x4 ra[4], rb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    ra[s] = operands[(threadIdx.x * 8 + s) % kProbeOperandPacks];
    rb[s] = operands[(threadIdx.x * 8 + 4 + s) % kProbeOperandPacks];
  }
  f32x4 acc[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) acc[t] = f32x4{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        bf16x8 a, b;
        __builtin_memcpy(&a, &ra[(s + t) & 3], 16);
        __builtin_memcpy(&b, &rb[(s + 3 * (t >> 2)) & 3], 16);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b, a, acc[t], 0, 0, 0);
      }
  }
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < 16; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) sum += acc[t][r];
  out[(size_t)blockIdx.x * kProbeThreads + threadIdx.x] = sum;
}

// MFMA work fed from LDS at the attention kernels' operand traffic: every
// v_mfma_f32_32x32x16_bf16 takes its first operand from one ds_read_b128 (1 KiB per
// wave: 16 bytes per lane, consecutive lanes on consecutive 16-byte chunks, no bank
// conflicts), the second from registers; two workgroups per CU (two waves per SIMD,
// as the attention kernels run). With EXP, one v_exp_f32 of an accumulator value per
// MFMA (the softmax's exponentials: the forward issues one per MFMA), of a scaled
// accumulator value so that the sum stays finite however large the accumulators grow
// (the operands repeat, so they grow with the iterations). 64 MFMAs per wave and
// iteration, as the register probe.
template <bool EXP>
__global__ __launch_bounds__(kProbeThreads, 2) void mfma_lds_probe_kernel(
    const u32x4* __restrict__ operands, float* __restrict__ out, int iters) {
  __shared__ u32x4 tile[kProbeOperandPacks];  // the 32 KiB of operands
  for (int i = threadIdx.x; i < kProbeOperandPacks; i += kProbeThreads) tile[i] = operands[i];
  __syncthreads();
  bf16x8 b[2];
  {
    const u32x4 t0 = operands[threadIdx.x % kProbeOperandPacks];
    const u32x4 t1 = operands[(threadIdx.x + 1024) % kProbeOperandPacks];
    __builtin_memcpy(&b[0], &t0, 16);
    __builtin_memcpy(&b[1], &t1, 16);
  }
  f32x16 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = f32x16{};
  float es = 0.f;
  int base = (int)threadIdx.x;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const u32x4 r = tile[(base + 64 * s) % kProbeOperandPacks];
        bf16x8 a;
        __builtin_memcpy(&a, &r, 16);
        acc[s & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[s & 1], acc[s & 3], 0, 0, 0);
      }
      if constexpr (EXP) {
#pragma unroll
        for (int e = 0; e < 16; ++e)
          es += __builtin_amdgcn_exp2f(__builtin_fmaf(acc[e & 3][e], 1e-30f, -1.0f));
      }
      base = (base + 17) % kProbeOperandPacks;
    }
  }
  float sum = es;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) sum += acc[t][r];
  out[(size_t)blockIdx.x * kProbeThreads + threadIdx.x] = sum;
}

}  // namespace
}  // namespace eg

using namespace eg;

extern "C" int eg_probe_mfma_bf16(const void* operands, float* out, int workgroups, int iters,
                                  void* stream) {
  clear_error();
  if (!operands || !out) {
    set_error("eg_probe_mfma_bf16: null pointer");
    return 1;
  }
  if (workgroups <= 0 || workgroups > 65536 || iters < 0) {
    set_error("eg_probe_mfma_bf16: workgroups must be in 1..65536 and iters non-negative");
    return 1;
  }
  if (!aligned16(operands)) {
    set_error("eg_probe_mfma_bf16: operands must be 16-byte aligned");
    return 1;
  }
  EG_LAUNCH(mfma_probe_kernel, dim3((unsigned)workgroups), dim3(kProbeThreads), 0,
            as_stream(stream), (const u32x4*)operands, out, iters);
  return check_launch("eg_probe_mfma_bf16");
}

extern "C" int eg_probe_mfma_mix(int kind, const void* operands, float* out, int workgroups,
                                 int iters, void* stream) {
  clear_error();
  if (!operands || !out) {
    set_error("eg_probe_mfma_mix: null pointer");
    return 1;
  }
  if (kind < 0 || kind > 3) {
    set_error("eg_probe_mfma_mix: kind must be 0 (32x32x16 from registers), 1 (16x16x32 from "
              "registers), 2 (32x32x16 with an LDS operand) or 3 (2 plus one exp per MFMA)");
    return 1;
  }
  if (workgroups <= 0 || workgroups > 65536 || iters < 0) {
    set_error("eg_probe_mfma_mix: workgroups must be in 1..65536 and iters non-negative");
    return 1;
  }
  if (!aligned16(operands)) {
    set_error("eg_probe_mfma_mix: operands must be 16-byte aligned");
    return 1;
  }
  const u32x4* ops = (const u32x4*)operands;
  hipStream_t st = as_stream(stream);
  switch (kind) {
    case 0: EG_LAUNCH(mfma_probe_kernel, dim3((unsigned)workgroups), dim3(kProbeThreads), 0, st, ops, out, iters); break;
    case 1: EG_LAUNCH(mfma16_probe_kernel, dim3((unsigned)workgroups), dim3(kProbeThreads), 0, st, ops, out, iters); break;
    case 2: EG_LAUNCH(mfma_lds_probe_kernel<false>, dim3((unsigned)workgroups), dim3(kProbeThreads), 0, st, ops, out, iters); break;
    default: EG_LAUNCH(mfma_lds_probe_kernel<true>, dim3((unsigned)workgroups), dim3(kProbeThreads), 0, st, ops, out, iters); break;
  }
  return check_launch("eg_probe_mfma_mix");
}
