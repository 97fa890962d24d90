// Row statistics over long rows, shared by the cross-entropy and the wide-row
// softmax kernels: a workgroup of BLOCK threads strides one row in VEC-element
// packs, kUnroll packs in flight per thread, and reduces over the workgroup with
// a fixed combine order (bitwise repeatable).
#pragma once

#include "eg_common.hpp"

namespace eg {
namespace rowwise {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kUnroll = 4;  // packs in flight per thread

// Reference point of a running max, as torch's logsumexp takes it: an infinite
// max is replaced by 0 so that exp(x - ref) stays defined.
__device__ __forceinline__ float lse_ref(float m) { return __builtin_isinf(m) ? 0.f : m; }

// logsumexp of the row xr[0 .. cols) in fp32, returned to every thread: an online
// (max, sum of exp2) per thread, then one max and one sum over the workgroup.
// `red` holds BLOCK / 64 floats of LDS.
template <typename T, int VEC, int BLOCK, bool NT>
__device__ __forceinline__ float row_lse(const T* __restrict__ xr, int cols, float* red) {
  constexpr int STEP = BLOCK * VEC;
  float m = -INFINITY;  // running max of this thread's elements
  float s = 0.f;        // sum of exp(v - lse_ref(m)) over them
  for (int base = (int)threadIdx.x * VEC; base < cols; base += STEP * kUnroll) {
    float v[kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = base + u * STEP;
      if (c < cols) {
        load_vec<T, VEC, NT>(xr + c, v[u]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[u][i] = -INFINITY;
      }
    }
    float bm = m;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int i = 0; i < VEC; ++i) bm = fmaxf(bm, v[u][i]);
    const float r_new = lse_ref(bm);
    const float rl = r_new * kLog2e;
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int i = 0; i < VEC; ++i)
        acc += __builtin_amdgcn_exp2f(__builtin_fmaf(v[u][i], kLog2e, -rl));
    // s == 0 also covers the first batch (m = -inf), where the rescale factor
    // could overflow.
    s = (s == 0.f) ? acc
                   : __builtin_fmaf(s, __builtin_amdgcn_exp2f((lse_ref(m) - r_new) * kLog2e),
                                    acc);
    m = bm;
  }
  const float gm = block_reduce<BLOCK>(m, MaxOp(), red);
  const float gref = lse_ref(gm);
  const float part =
      (s == 0.f) ? 0.f : s * __builtin_amdgcn_exp2f((lse_ref(m) - gref) * kLog2e);
  const float total = block_reduce<BLOCK>(part, SumOp(), red);
  return gref + log2f(total) * kLn2;
}

// sum(a * b) over the row, in fp32, returned to every thread.
template <typename T, int VEC, int BLOCK, bool NT>
__device__ __forceinline__ float row_dot(const T* __restrict__ a, const T* __restrict__ b,
                                         int cols, float* red) {
  constexpr int STEP = BLOCK * VEC;
  float d = 0.f;
  for (int base = (int)threadIdx.x * VEC; base < cols; base += STEP * kUnroll) {
    float va[kUnroll][VEC], vb[kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = base + u * STEP;
      if (c < cols) {
        load_vec<T, VEC, NT>(a + c, va[u]);
        load_vec<T, VEC, NT>(b + c, vb[u]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) va[u][i] = vb[u][i] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int i = 0; i < VEC; ++i) d += va[u][i] * vb[u][i];
  }
  return block_reduce<BLOCK>(d, SumOp(), red);
}

// Smallest power-of-two workgroup (64..1024 threads) whose threads cover a row of
// `npack` packs in one pass of kUnroll packs each.
template <typename Launch>
void pick_row_block(int64_t npack, Launch&& launch) {
  const int64_t per = (npack + kUnroll - 1) / kUnroll;
  if (per <= 64) launch.template go<64>();
  else if (per <= 128) launch.template go<128>();
  else if (per <= 256) launch.template go<256>();
  else if (per <= 512) launch.template go<512>();
  else launch.template go<1024>();
}

// Elementwise passes over a row-major [rows, cols] matrix as one flat sequence of
// packs: workgroup b covers packs [b * kFlatPer, (b + 1) * kFlatPer) in address
// order, so the workgroups in flight stream through contiguous memory. With at
// least kFlatPer packs per row a workgroup spans at most two rows.
constexpr int kFlatBlock = 512;
constexpr int kFlatUnroll = 2;
constexpr int kFlatPer = kFlatBlock * kFlatUnroll;

}  // namespace rowwise
}  // namespace eg
