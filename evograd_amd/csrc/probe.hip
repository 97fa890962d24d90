// Sustained bf16 MFMA rate of the device, as a measurement aid for the roofline
// figures: the published dense peak (2516.6 TFLOP/s) assumes the 2.4 GHz engine
// clock, which the device holds only while the matrix cores see low-toggle data;
// with random bf16 operands power management lowers the clock. This kernel keeps
// every SIMD's matrix core busy from registers alone (no memory traffic inside
// the loop), on operands the caller fills with random bf16 values, so its rate is
// the ceiling a kernel's MFMA work can approach on this device.
#include "eg_common.hpp"

namespace eg {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
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
