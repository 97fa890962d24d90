// Row softmax forward/backward for gfx950.
//
// Forward follows softmax_forward_ref (src/evograd/ops/level1/softmax/forward_ref.py:6-7):
// y = exp(x - max) / sum(exp(x - max)) in fp32, cast to the I/O dtype. Backward is
// the rule declared at src/evograd/ops/level1/softmax/__init__.py:78:
// dx = y * (dy - sum(dy * y)).
//
// One workgroup per row. When the row fits in registers (BLOCK threads x ITEMS
// packs x VEC elements >= cols) it is read from HBM exactly once with 16-byte
// loads, reduced with wave butterflies + one LDS exchange, and written once.
// 16-bit rows up to 131072 columns keep the forward's x, and the backward's y, in
// registers as raw packs (softmax_fwd_raw / softmax_bwd_raw). Wider rows take a
// two-read path: the row's logsumexp
// (forward) or sum(dy * y) (backward) in one read, then y = exp(x - lse) or
// dx = y * (dy - sum) in a second read and the write.
#include "rowwise.hpp"

namespace eg {
namespace {

template <typename T, int VEC, int ITEMS, int BLOCK, bool NT>
__device__ __forceinline__ void load_row(const T* __restrict__ row, int cols, float fill,
                                         float (&v)[ITEMS][VEC]) {
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
    if (c < cols) {
      load_vec<T, VEC, NT>(row + c, v[it]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) v[it][i] = fill;
    }
  }
}

template <typename T, int VEC, int ITEMS, int BLOCK, bool NT>
__device__ __forceinline__ void store_row(T* __restrict__ row, int cols,
                                          const float (&v)[ITEMS][VEC]) {
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
    if (c < cols) store_vec<T, VEC, NT>(row + c, v[it]);
  }
}

template <typename T, int VEC, int ITEMS, int BLOCK, bool NT>
__global__ __launch_bounds__(BLOCK) void softmax_fwd_reg(const T* __restrict__ x,
                                                         T* __restrict__ y, int cols) {
  __shared__ float lds[BLOCK / kWave];
  const int64_t off = (int64_t)blockIdx.x * cols;
  float v[ITEMS][VEC];
  load_row<T, VEC, ITEMS, BLOCK, NT>(x + off, cols, -INFINITY, v);
  float m = -INFINITY;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) m = fmaxf(m, v[it][i]);
  m = block_reduce<BLOCK>(m, MaxOp(), lds);
  float s = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      v[it][i] = expf(v[it][i] - m);
      s += v[it][i];
    }
  s = block_reduce<BLOCK>(s, SumOp(), lds);
  const float inv = 1.0f / s;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[it][i] *= inv;
  store_row<T, VEC, ITEMS, BLOCK, NT>(y + off, cols, v);
}

template <typename T, int VEC, int ITEMS, int BLOCK, bool NT>
__global__ __launch_bounds__(BLOCK) void softmax_bwd_reg(const T* __restrict__ y,
                                                         const T* __restrict__ dy,
                                                         T* __restrict__ dx, int cols) {
  __shared__ float lds[BLOCK / kWave];
  const int64_t off = (int64_t)blockIdx.x * cols;
  float yv[ITEMS][VEC], gv[ITEMS][VEC];
  load_row<T, VEC, ITEMS, BLOCK, NT>(y + off, cols, 0.f, yv);
  load_row<T, VEC, ITEMS, BLOCK, NT>(dy + off, cols, 0.f, gv);
  float d = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) d += gv[it][i] * yv[it][i];
  d = block_reduce<BLOCK>(d, SumOp(), lds);
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) gv[it][i] = yv[it][i] * (gv[it][i] - d);
  store_row<T, VEC, ITEMS, BLOCK, NT>(dx + off, cols, gv);
}

// ---- wide rows: one read for the row statistic (lse, or sum(dy * y)), a second
// read to write, each with kUnroll 16-byte packs in flight per thread.
template <typename T, int VEC, int BLOCK, bool NT>
__global__ __launch_bounds__(BLOCK) void softmax_fwd_loop(const T* __restrict__ x,
                                                          T* __restrict__ y, int cols) {
  __shared__ float lds[BLOCK / kWave];
  constexpr int STEP = BLOCK * VEC;
  const int64_t off = (int64_t)blockIdx.x * cols;
  const T* __restrict__ xr = x + off;
  T* __restrict__ yr = y + off;
  // y = exp(x - lse): the max and the normaliser folded into one reference point.
  // The statistic's read is a temporal load, so that the rows in flight (256 KB
  // each at bf16 x 128K columns) can serve the second read from the device cache;
  // the second read is the last use.
  const float ll = rowwise::row_lse<T, VEC, BLOCK, false>(xr, cols, lds) * rowwise::kLog2e;
  for (int base = (int)threadIdx.x * VEC; base < cols; base += STEP * rowwise::kUnroll) {
    float v[rowwise::kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < rowwise::kUnroll; ++u) {
      const int c = base + u * STEP;
      if (c < cols) load_vec<T, VEC, NT>(xr + c, v[u]);
    }
#pragma unroll
    for (int u = 0; u < rowwise::kUnroll; ++u) {
      const int c = base + u * STEP;
      if (c < cols) {
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          v[u][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(v[u][i], rowwise::kLog2e, -ll));
        store_vec<T, VEC, NT>(yr + c, v[u]);
      }
    }
  }
}

template <typename T, int VEC, int BLOCK, bool NT>
__global__ __launch_bounds__(BLOCK) void softmax_bwd_loop(const T* __restrict__ y,
                                                          const T* __restrict__ dy,
                                                          T* __restrict__ dx, int cols) {
  __shared__ float lds[BLOCK / kWave];
  constexpr int STEP = BLOCK * VEC;
  const int64_t off = (int64_t)blockIdx.x * cols;
  const T* __restrict__ yr = y + off;
  const T* __restrict__ gr = dy + off;
  T* __restrict__ dr = dx + off;
  // temporal first read, as in the forward
  const float d = rowwise::row_dot<T, VEC, BLOCK, false>(yr, gr, cols, lds);
  for (int base = (int)threadIdx.x * VEC; base < cols; base += STEP * rowwise::kUnroll) {
    float a[rowwise::kUnroll][VEC], b[rowwise::kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < rowwise::kUnroll; ++u) {
      const int c = base + u * STEP;
      if (c < cols) {
        load_vec<T, VEC, NT>(yr + c, a[u]);
        load_vec<T, VEC, NT>(gr + c, b[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < rowwise::kUnroll; ++u) {
      const int c = base + u * STEP;
      if (c < cols) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) b[u][i] = a[u][i] * (b[u][i] - d);
        store_vec<T, VEC, NT>(dr + c, b[u]);
      }
    }
  }
}

// ---- 16-bit rows up to 16 packs x 1024 threads (131072 columns, the Llama-3
// vocabulary): the row stays in registers as raw 16-byte packs (64 VGPRs) and is
// converted again in each pass, so it is read from HBM once. The empty asm
// statements keep the compiler from hoisting fp32 copies of the row (128 VGPRs,
// which would spill at 1024 threads).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ void unpack8(const u32x4& raw, float (&f)[8]) {
  Pack<T, 8> pk;
  __builtin_memcpy(&pk, &raw, 16);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = to_f32(pk.v[i]);
}

template <typename T, int ITEMS, int BLOCK>
__global__ __launch_bounds__(BLOCK) void softmax_fwd_raw(const T* __restrict__ x,
                                                         T* __restrict__ y, int cols) {
  static_assert(sizeof(T) == 2, "raw rows hold 16-bit elements");
  __shared__ float lds[BLOCK / kWave];
  const int64_t off = (int64_t)blockIdx.x * cols;
  u32x4 raw[ITEMS];
  u32x4 fill;
  {
    Pack<T, 8> pk;
#pragma unroll
    for (int i = 0; i < 8; ++i) pk.v[i] = from_f32<T>(-INFINITY);
    __builtin_memcpy(&fill, &pk, 16);
  }
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * 8;
    raw[it] = c < cols ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + off + c))
                       : fill;
  }
  float m = -INFINITY;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    float f[8];
    unpack8<T>(raw[it], f);
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, f[i]);
  }
  m = block_reduce<BLOCK>(m, MaxOp(), lds);
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) asm volatile("" : "+v"(raw[it]));
  const float ml = m * rowwise::kLog2e;
  float s = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    float f[8];
    unpack8<T>(raw[it], f);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      s += __builtin_amdgcn_exp2f(__builtin_fmaf(f[i], rowwise::kLog2e, -ml));
  }
  s = block_reduce<BLOCK>(s, SumOp(), lds);
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) asm volatile("" : "+v"(raw[it]));
  const float ll = ml + log2f(s);  // log2 of the row's normaliser, max included
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * 8;
    if (c < cols) {
      float f[8];
      unpack8<T>(raw[it], f);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        f[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(f[i], rowwise::kLog2e, -ll));
      store_vec<T, 8, true>(y + off + c, f);
    }
  }
}
constexpr int kRawItems = 16, kRawBlock = 1024;

// Backward for the same rows: y stays in registers as raw packs, dy is read twice
// (the first read temporal, so the rows in flight serve the second from the
// device cache): sum(dy * y), then dx = y * (dy - sum).
template <typename T, int ITEMS, int BLOCK>
__global__ __launch_bounds__(BLOCK) void softmax_bwd_raw(const T* __restrict__ y,
                                                         const T* __restrict__ dy,
                                                         T* __restrict__ dx, int cols) {
  static_assert(sizeof(T) == 2, "raw rows hold 16-bit elements");
  __shared__ float lds[BLOCK / kWave];
  const int64_t off = (int64_t)blockIdx.x * cols;
  u32x4 raw[ITEMS];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * 8;
    raw[it] = c < cols ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(y + off + c))
                       : u32x4{0u, 0u, 0u, 0u};
  }
  float d = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * 8;
    if (c < cols) {
      float f[8], g[8];
      unpack8<T>(raw[it], f);
      load_vec<T, 8, false>(dy + off + c, g);
#pragma unroll
      for (int i = 0; i < 8; ++i) d += f[i] * g[i];
    }
  }
  d = block_reduce<BLOCK>(d, SumOp(), lds);
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) asm volatile("" : "+v"(raw[it]));
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * 8;
    if (c < cols) {
      float f[8], g[8];
      unpack8<T>(raw[it], f);
      load_vec<T, 8, true>(dy + off + c, g);
#pragma unroll
      for (int i = 0; i < 8; ++i) g[i] = f[i] * (g[i] - d);
      store_vec<T, 8, true>(dx + off + c, g);
    }
  }
}

// Picks (BLOCK, ITEMS) so that BLOCK * ITEMS packs cover the row; returns false
// when the row is too wide for the register path.
template <typename Launch>
bool pick_row_config(int64_t npack, Launch&& launch) {
  if (npack <= 64) return launch.template go<64, 1>();
  if (npack <= 128) return launch.template go<128, 1>();
  if (npack <= 256) return launch.template go<256, 1>();
  if (npack <= 512) return launch.template go<256, 2>();
  if (npack <= 1024) return launch.template go<256, 4>();
  if (npack <= 2048) return launch.template go<512, 4>();
  if (npack <= 4096) return launch.template go<1024, 4>();
  if (npack <= 8192) return launch.template go<1024, 8>();
  return false;
}

template <typename T, int VEC>
struct FwdLaunch {
  const T* x; T* y; int64_t rows; int cols; hipStream_t st;
  template <int BLOCK, int ITEMS> bool go() {
    EG_LAUNCH((softmax_fwd_reg<T, VEC, ITEMS, BLOCK, VEC * sizeof(T) == 16>), dim3((unsigned)rows),
                       dim3(BLOCK), 0, st, x, y, cols);
    return true;
  }
};

template <typename T, int VEC>
struct BwdLaunch {
  const T* y; const T* dy; T* dx; int64_t rows; int cols; hipStream_t st;
  template <int BLOCK, int ITEMS> bool go() {
    EG_LAUNCH((softmax_bwd_reg<T, VEC, ITEMS, BLOCK, VEC * sizeof(T) == 16>), dim3((unsigned)rows),
                       dim3(BLOCK), 0, st, y, dy, dx, cols);
    return true;
  }
};

template <typename T, int VEC>
void softmax_fwd_vec(const T* x, T* y, int64_t rows, int cols, hipStream_t st) {
  FwdLaunch<T, VEC> l{x, y, rows, cols, st};
  const int64_t npack = (cols + VEC - 1) / VEC;
  if (pick_row_config(npack, l)) return;
  if constexpr (sizeof(T) == 2 && VEC == 8) {
    if (npack <= (int64_t)kRawItems * kRawBlock) {
      EG_LAUNCH((softmax_fwd_raw<T, kRawItems, kRawBlock>), dim3((unsigned)rows), dim3(kRawBlock),
                0, st, x, y, cols);
      return;
    }
  }
  EG_LAUNCH((softmax_fwd_loop<T, VEC, 1024, VEC * sizeof(T) == 16>), dim3((unsigned)rows),
            dim3(1024), 0, st, x, y, cols);
}

template <typename T, int VEC>
void softmax_bwd_vec(const T* y, const T* dy, T* dx, int64_t rows, int cols, hipStream_t st) {
  BwdLaunch<T, VEC> l{y, dy, dx, rows, cols, st};
  const int64_t npack = (cols + VEC - 1) / VEC;
  if (pick_row_config(npack, l)) return;
  if constexpr (sizeof(T) == 2 && VEC == 8) {
    if (npack <= (int64_t)kRawItems * kRawBlock) {
      EG_LAUNCH((softmax_bwd_raw<T, kRawItems, kRawBlock>), dim3((unsigned)rows), dim3(kRawBlock),
                0, st, y, dy, dx, cols);
      return;
    }
  }
  EG_LAUNCH((softmax_bwd_loop<T, VEC, 1024, VEC * sizeof(T) == 16>), dim3((unsigned)rows),
            dim3(1024), 0, st, y, dy, dx, cols);
}

int check_dims(const char* what, int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) {
    set_error("%s: negative size rows=%lld cols=%lld", what, (long long)rows, (long long)cols);
    return 1;
  }
  if (cols > (int64_t)1 << 30 || rows > (int64_t)0x7fffffff) {
    set_error("%s: size out of range rows=%lld cols=%lld", what, (long long)rows,
              (long long)cols);
    return 1;
  }
  return 0;
}

}  // namespace
}  // namespace eg

using namespace eg;

extern "C" int eg_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, int dtype,
                              void* stream) {
  clear_error();
  if (check_dims("eg_softmax_fwd", rows, cols)) return 1;
  if (rows == 0 || cols == 0) return 0;
  if (!x || !y) { set_error("eg_softmax_fwd: null pointer"); return 1; }
  hipStream_t st = as_stream(stream);
  return EG_DISPATCH_FLOAT(dtype, "eg_softmax_fwd", [&] {
    using T = scalar_t;
    constexpr int V = 16 / sizeof(T);
    const T* xp = static_cast<const T*>(x);
    T* yp = static_cast<T*>(y);
    if (cols % V == 0 && aligned16(x) && aligned16(y))
      softmax_fwd_vec<T, V>(xp, yp, rows, (int)cols, st);
    else
      softmax_fwd_vec<T, 1>(xp, yp, rows, (int)cols, st);
    return check_launch("eg_softmax_fwd");
  });
}

extern "C" int eg_softmax_bwd(const void* y, const void* dy, void* dx, int64_t rows,
                              int64_t cols, int dtype, void* stream) {
  clear_error();
  if (check_dims("eg_softmax_bwd", rows, cols)) return 1;
  if (rows == 0 || cols == 0) return 0;
  if (!y || !dy || !dx) { set_error("eg_softmax_bwd: null pointer"); return 1; }
  hipStream_t st = as_stream(stream);
  return EG_DISPATCH_FLOAT(dtype, "eg_softmax_bwd", [&] {
    using T = scalar_t;
    constexpr int V = 16 / sizeof(T);
    const T* yp = static_cast<const T*>(y);
    const T* gp = static_cast<const T*>(dy);
    T* dp = static_cast<T*>(dx);
    if (cols % V == 0 && aligned16(y) && aligned16(dy) && aligned16(dx))
      softmax_bwd_vec<T, V>(yp, gp, dp, rows, (int)cols, st);
    else
      softmax_bwd_vec<T, 1>(yp, gp, dp, rows, (int)cols, st);
    return check_launch("eg_softmax_bwd");
  });
}
