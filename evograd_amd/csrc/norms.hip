// RMSNorm and LayerNorm forward/backward for gfx950.
//
// RMSNorm follows rmsnorm_forward_ref (src/evograd/ops/level1/rmsnorm/forward_ref.py:6-21)
// and the backward rule at src/evograd/ops/level1/rmsnorm/__init__.py:85-86.
// LayerNorm follows layernorm_forward_ref (src/evograd/ops/level1/layernorm/forward_ref.py:6-23)
// and its autograd backward (grads declared at layernorm/__init__.py:124-171).
//
// Layout: x, y, dy, dx are [rows, hidden] row-major in HBM; weight/bias [hidden];
// the saved statistics (rstd, and mean for LayerNorm) are fp32 [rows].
//
// Forward: one wave per row when the row is 1..8 packs per lane (RMSNorm), else
// one workgroup per row; the row is held in registers (16-byte packs) and its
// statistics reduced by wave butterflies (and one LDS exchange for workgroups).
//
// Backward: G = min(rows, kPartialBlocks) workgroups walk the rows with stride G.
// Each thread owns a fixed set of columns for the whole walk, so it keeps its
// weight values and its dweight (and dbias) accumulators in registers; the next
// row's loads are issued before the current row is reduced. At the end every
// workgroup writes one fp32 partial row to the workspace [G, hidden], and a small
// kernel sums the G partials per column in a fixed order. No atomics: the result
// is bit-identical from run to run.
#include "eg_common.hpp"

#include <initializer_list>

namespace eg {
namespace {

constexpr int kPartialBlocks = 512;

inline int64_t partial_blocks(int64_t rows) {
  return rows < kPartialBlocks ? (rows > 0 ? rows : 1) : kPartialBlocks;
}

template <typename T, int VEC, int ITEMS, int BLOCK, bool NT = false>
__device__ __forceinline__ void load_cols(const T* __restrict__ p, int n, float (&v)[ITEMS][VEC]) {
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
    if (c < n) {
      load_vec<T, VEC, NT>(p + c, v[it]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) v[it][i] = 0.f;
    }
  }
}

template <typename T, int VEC, int ITEMS, int BLOCK, bool NT = false>
__device__ __forceinline__ void store_cols(T* __restrict__ p, int n, const float (&v)[ITEMS][VEC]) {
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
    if (c < n) store_vec<T, VEC, NT>(p + c, v[it]);
  }
}

// ------------------------------------------------------------------ RMSNorm
template <typename T, int VEC, int ITEMS, int BLOCK, bool NT>
__global__ __launch_bounds__(BLOCK) void rmsnorm_fwd_kernel(const T* __restrict__ x,
                                                            const T* __restrict__ w,
                                                            T* __restrict__ y,
                                                            float* __restrict__ rstd_out,
                                                            int hidden, float eps) {
  __shared__ float lds[BLOCK / kWave];
  const int64_t row = blockIdx.x;
  const int64_t off = row * hidden;
  float xv[ITEMS][VEC], wv[ITEMS][VEC];
  load_cols<T, VEC, ITEMS, BLOCK, NT>(x + off, hidden, xv);
  load_cols<T, VEC, ITEMS, BLOCK>(w, hidden, wv);
  float ss = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) ss += xv[it][i] * xv[it][i];
  ss = block_reduce<BLOCK>(ss, SumOp(), lds);
  const float rstd = rsqrtf(ss / (float)hidden + eps);
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) xv[it][i] = (xv[it][i] * rstd) * wv[it][i];
  store_cols<T, VEC, ITEMS, BLOCK, NT>(y + off, hidden, xv);
  if (threadIdx.x == 0) rstd_out[row] = rstd;
}

template <typename T, int VEC, int ITEMS, int BLOCK, bool NT>
__global__ __launch_bounds__(BLOCK) void rmsnorm_bwd_kernel(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ w,
    const float* __restrict__ rstd, T* __restrict__ dx, float* __restrict__ partial,
    int64_t rows, int hidden) {
  __shared__ float lds[BLOCK / kWave];
  const int64_t G = gridDim.x;
  float wv[ITEMS][VEC], acc[ITEMS][VEC];
  load_cols<T, VEC, ITEMS, BLOCK>(w, hidden, wv);
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[it][i] = 0.f;
  const float inv_h = 1.0f / (float)hidden;

  int64_t row = blockIdx.x;
  float xv[ITEMS][VEC], gv[ITEMS][VEC];
  float r = 0.f;
  if (row < rows) {
    load_cols<T, VEC, ITEMS, BLOCK, NT>(x + row * hidden, hidden, xv);
    load_cols<T, VEC, ITEMS, BLOCK, NT>(dy + row * hidden, hidden, gv);
    r = rstd[row];
  }
  while (row < rows) {
    // Prefetch the next row of this workgroup while the current one reduces.
    const int64_t nrow = row + G;
    float nx[ITEMS][VEC], ng[ITEMS][VEC];
    float nr = 0.f;
    if (nrow < rows) {
      load_cols<T, VEC, ITEMS, BLOCK, NT>(x + nrow * hidden, hidden, nx);
      load_cols<T, VEC, ITEMS, BLOCK, NT>(dy + nrow * hidden, hidden, ng);
      nr = rstd[nrow];
    }
    float dot = 0.f;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it)
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float xh = xv[it][i] * r;
        acc[it][i] += gv[it][i] * xh;
        const float g = gv[it][i] * wv[it][i];
        xv[it][i] = xh;
        gv[it][i] = g;
        dot += g * xh;
      }
    dot = block_reduce<BLOCK>(dot, SumOp(), lds) * inv_h;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it)
#pragma unroll
      for (int i = 0; i < VEC; ++i) gv[it][i] = (gv[it][i] - xv[it][i] * dot) * r;
    store_cols<T, VEC, ITEMS, BLOCK, NT>(dx + row * hidden, hidden, gv);
    row = nrow;
    if (row < rows) {
#pragma unroll
      for (int it = 0; it < ITEMS; ++it)
#pragma unroll
        for (int i = 0; i < VEC; ++i) { xv[it][i] = nx[it][i]; gv[it][i] = ng[it][i]; }
      r = nr;
    }
  }
  float* pp = partial + (int64_t)blockIdx.x * hidden;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
    if (c < hidden) store_f32<float, VEC>(pp + c, acc[it]);
  }
}

// --------------------------------------------- RMSNorm forward, one wave per row
// For rows of ITEMS x 64 lanes x VEC elements (hidden 512..4096 in bf16) a wave
// owns a whole row: the statistic is reduced with wave butterflies only, so no
// workgroup barrier sits between a row's loads and its stores, and the waves of a
// CU drift independently, keeping many rows of loads in flight. (The same shape
// for the backward, with per-lane dweight sums, measured slower than the
// workgroup kernel below and is not used.)
template <typename T, int VEC>
__device__ __forceinline__ Pack<T, VEC> ld_pack(const T* __restrict__ p) {
  static_assert(sizeof(T) * VEC == 16, "16-byte packs");
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  Pack<T, VEC> pk;
  __builtin_memcpy(&pk, &raw, 16);
  return pk;
}

template <typename T, int VEC, int ITEMS>
__global__ __launch_bounds__(256) void rmsnorm_fwd_wave(const T* __restrict__ x,
                                                        const T* __restrict__ w,
                                                        T* __restrict__ y,
                                                        float* __restrict__ rstd_out, int64_t rows,
                                                        float eps) {
  constexpr int H = ITEMS * kWave * VEC;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * H;
  Pack<T, VEC> xp[ITEMS];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) xp[it] = ld_pack<T, VEC>(xr + (it * kWave + lane) * VEC);
  float ss = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float v = to_f32(xp[it].v[i]);
      ss += v * v;
    }
  ss = wave_reduce(ss, SumOp());
  const float r = rsqrtf(ss / (float)H + eps);
  T* yr = y + row * H;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * kWave + lane) * VEC;
    const Pack<T, VEC> wp = *reinterpret_cast<const Pack<T, VEC>*>(w + c);
    float o[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) o[i] = (to_f32(xp[it].v[i]) * r) * to_f32(wp.v[i]);
    store_f32_nt<T, VEC>(yr + c, o);
  }
  if (lane == 0) rstd_out[row] = r;
}

// ---------------------------------------------------------------- LayerNorm
template <typename T, int VEC, int ITEMS, int BLOCK, bool NT>
__global__ __launch_bounds__(BLOCK) void layernorm_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ b,
    T* __restrict__ y, float* __restrict__ mean_out, float* __restrict__ rstd_out,
    int hidden, float eps) {
  __shared__ float lds[BLOCK / kWave];
  const int64_t row = blockIdx.x;
  const int64_t off = row * hidden;
  float xv[ITEMS][VEC];
  load_cols<T, VEC, ITEMS, BLOCK, NT>(x + off, hidden, xv);
  float s = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) s += xv[it][i];
  const float mean = block_reduce<BLOCK>(s, SumOp(), lds) / (float)hidden;
  float q = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float d = (c + i < hidden) ? xv[it][i] - mean : 0.f;
      q += d * d;
    }
  }
  const float var = block_reduce<BLOCK>(q, SumOp(), lds) / (float)hidden;
  const float rstd = rsqrtf(var + eps);
  float wv[ITEMS][VEC], bv[ITEMS][VEC];
  load_cols<T, VEC, ITEMS, BLOCK>(w, hidden, wv);
  load_cols<T, VEC, ITEMS, BLOCK>(b, hidden, bv);
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i)
      xv[it][i] = ((xv[it][i] - mean) * rstd) * wv[it][i] + bv[it][i];
  store_cols<T, VEC, ITEMS, BLOCK, NT>(y + off, hidden, xv);
  if (threadIdx.x == 0) { mean_out[row] = mean; rstd_out[row] = rstd; }
}

template <typename T, int VEC, int ITEMS, int BLOCK, bool NT>
__global__ __launch_bounds__(BLOCK) void layernorm_bwd_kernel(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ w,
    const float* __restrict__ mean, const float* __restrict__ rstd, T* __restrict__ dx,
    float* __restrict__ partial_w, float* __restrict__ partial_b, int64_t rows, int hidden) {
  __shared__ float lds[2 * (BLOCK / kWave)];
  const int64_t G = gridDim.x;
  float wv[ITEMS][VEC], accw[ITEMS][VEC], accb[ITEMS][VEC];
  load_cols<T, VEC, ITEMS, BLOCK>(w, hidden, wv);
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) { accw[it][i] = 0.f; accb[it][i] = 0.f; }
  const float inv_h = 1.0f / (float)hidden;

  int64_t row = blockIdx.x;
  float xv[ITEMS][VEC], gv[ITEMS][VEC];
  float mu = 0.f, r = 0.f;
  if (row < rows) {
    load_cols<T, VEC, ITEMS, BLOCK, NT>(x + row * hidden, hidden, xv);
    load_cols<T, VEC, ITEMS, BLOCK, NT>(dy + row * hidden, hidden, gv);
    mu = mean[row];
    r = rstd[row];
  }
  while (row < rows) {
    const int64_t nrow = row + G;
    float nx[ITEMS][VEC], ng[ITEMS][VEC];
    float nmu = 0.f, nr = 0.f;
    if (nrow < rows) {
      load_cols<T, VEC, ITEMS, BLOCK, NT>(x + nrow * hidden, hidden, nx);
      load_cols<T, VEC, ITEMS, BLOCK, NT>(dy + nrow * hidden, hidden, ng);
      nmu = mean[nrow];
      nr = rstd[nrow];
    }
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        // Padding columns load zeros for x but must also give xhat = 0.
        const float xh = (c + i < hidden) ? (xv[it][i] - mu) * r : 0.f;
        accw[it][i] += gv[it][i] * xh;
        accb[it][i] += gv[it][i];
        const float g = gv[it][i] * wv[it][i];
        xv[it][i] = xh;
        gv[it][i] = g;
        sg += g;
        sgx += g * xh;
      }
    }
    block_reduce2<BLOCK>(sg, sgx, lds);
    sg *= inv_h;
    sgx *= inv_h;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it)
#pragma unroll
      for (int i = 0; i < VEC; ++i) gv[it][i] = r * ((gv[it][i] - sg) - xv[it][i] * sgx);
    store_cols<T, VEC, ITEMS, BLOCK, NT>(dx + row * hidden, hidden, gv);
    row = nrow;
    if (row < rows) {
#pragma unroll
      for (int it = 0; it < ITEMS; ++it)
#pragma unroll
        for (int i = 0; i < VEC; ++i) { xv[it][i] = nx[it][i]; gv[it][i] = ng[it][i]; }
      mu = nmu;
      r = nr;
    }
  }
  float* pw = partial_w + (int64_t)blockIdx.x * hidden;
  float* pb = partial_b + (int64_t)blockIdx.x * hidden;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
    if (c < hidden) {
      store_f32<float, VEC>(pw + c, accw[it]);
      store_f32<float, VEC>(pb + c, accb[it]);
    }
  }
}

// ------------------------------------------------- stage 2: column sums
// out[p][c] = sum_{g=0..G-1} partial[p][g][c] in a fixed order. A workgroup owns
// 64 columns (16 lanes x 4 columns); its 16 row groups each sum the partial rows
// g = rg, rg + 16, ... in ascending order with all loads of a batch issued
// together, and the 16 group totals are then added in group order through LDS.
// blockIdx.y selects the parameter (dweight, dbias).
constexpr int kColGroups = 16;
constexpr int kColBatch = 16;

template <typename T>
__global__ __launch_bounds__(256) void colsum_kernel(const float* __restrict__ partial,
                                                     T* __restrict__ o0, T* __restrict__ o1,
                                                     int G, int hidden) {
  __shared__ float4 lds[kColGroups][16];
  const int q = threadIdx.x & 15;   // column quad within the tile
  const int rg = threadIdx.x >> 4;  // row group
  const int c = blockIdx.x * 64 + 4 * q;
  const float* p = partial + (int64_t)blockIdx.y * G * hidden;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (c + 3 < hidden && (hidden & 3) == 0) {
    for (int g0 = rg; g0 < G; g0 += kColGroups * kColBatch) {
      float4 v[kColBatch];
#pragma unroll
      for (int i = 0; i < kColBatch; ++i) {
        const int g = g0 + i * kColGroups;
        v[i] = g < G ? *reinterpret_cast<const float4*>(p + (int64_t)g * hidden + c)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int i = 0; i < kColBatch; ++i) {
        acc.x += v[i].x; acc.y += v[i].y; acc.z += v[i].z; acc.w += v[i].w;
      }
    }
  } else {
    float a4[4] = {0.f, 0.f, 0.f, 0.f};
    for (int g = rg; g < G; g += kColGroups)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c + i < hidden) a4[i] += p[(int64_t)g * hidden + c + i];
    acc = make_float4(a4[0], a4[1], a4[2], a4[3]);
  }
  lds[rg][q] = acc;
  __syncthreads();
  if (rg == 0) {
    float4 t = lds[0][q];
#pragma unroll
    for (int r = 1; r < kColGroups; ++r) {
      const float4 u = lds[r][q];
      t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
    }
    T* o = blockIdx.y == 0 ? o0 : o1;
    const float tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (c + i < hidden) o[c + i] = from_f32<T>(tv[i]);
  }
}

template <typename T>
int launch_colsum(const float* partial, T* o0, T* o1, int nparams, int G, int hidden,
                  hipStream_t st, const char* what) {
  hipLaunchKernelGGL((colsum_kernel<T>), dim3((unsigned)((hidden + 63) / 64), (unsigned)nparams),
                     dim3(256), 0, st, partial, o0, o1, G, hidden);
  return check_launch(what);
}

// ------------------------------------------------------------- dispatch
template <typename F>
bool pick_norm_config(int64_t npack, F&& f) {
  if (npack <= 64) return f.template go<64, 1>();
  if (npack <= 128) return f.template go<128, 1>();
  if (npack <= 256) return f.template go<256, 1>();
  if (npack <= 512) return f.template go<512, 1>();
  if (npack <= 1024) return f.template go<512, 2>();
  if (npack <= 2048) return f.template go<1024, 2>();
  if (npack <= 4096) return f.template go<1024, 4>();
  if (npack <= 8192) return f.template go<1024, 8>();
  return false;
}

template <typename T, int VEC>
struct RmsFwd {
  const T *x, *w; T* y; float* rstd; int64_t rows; int hidden; float eps; hipStream_t st;
  template <int BLOCK, int ITEMS> bool go() {
    hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, VEC, ITEMS, BLOCK, VEC * sizeof(T) == 16>), dim3((unsigned)rows),
                       dim3(BLOCK), 0, st, x, w, y, rstd, hidden, eps);
    return true;
  }
};

template <typename T, int VEC>
struct RmsBwd {
  const T *dy, *x, *w; const float* rstd; T* dx; float* part; int64_t rows; int hidden;
  hipStream_t st;
  template <int BLOCK, int ITEMS> bool go() {
    hipLaunchKernelGGL((rmsnorm_bwd_kernel<T, VEC, ITEMS, BLOCK, VEC * sizeof(T) == 16>),
                       dim3((unsigned)partial_blocks(rows)), dim3(BLOCK), 0, st, dy, x, w, rstd,
                       dx, part, rows, hidden);
    return true;
  }
};

template <typename T, int VEC>
struct LnFwd {
  const T *x, *w, *b; T* y; float *mean, *rstd; int64_t rows; int hidden; float eps;
  hipStream_t st;
  template <int BLOCK, int ITEMS> bool go() {
    hipLaunchKernelGGL((layernorm_fwd_kernel<T, VEC, ITEMS, BLOCK, VEC * sizeof(T) == 16>), dim3((unsigned)rows),
                       dim3(BLOCK), 0, st, x, w, b, y, mean, rstd, hidden, eps);
    return true;
  }
};

template <typename T, int VEC>
struct LnBwd {
  const T *dy, *x, *w; const float *mean, *rstd; T* dx; float *pw, *pb; int64_t rows;
  int hidden; hipStream_t st;
  template <int BLOCK, int ITEMS> bool go() {
    hipLaunchKernelGGL((layernorm_bwd_kernel<T, VEC, ITEMS, BLOCK, VEC * sizeof(T) == 16>),
                       dim3((unsigned)partial_blocks(rows)), dim3(BLOCK), 0, st, dy, x, w, mean,
                       rstd, dx, pw, pb, rows, hidden);
    return true;
  }
};

int check_norm_dims(const char* what, int64_t rows, int64_t hidden) {
  if (rows < 0 || hidden <= 0) {
    set_error("%s: bad size rows=%lld hidden=%lld", what, (long long)rows, (long long)hidden);
    return 1;
  }
  if (rows > (int64_t)0x7fffffff || hidden > 8192 * 8) {
    set_error("%s: size out of range rows=%lld hidden=%lld", what, (long long)rows,
              (long long)hidden);
    return 1;
  }
  return 0;
}

template <typename T>
bool vec_ok(int hidden, std::initializer_list<const void*> ptrs) {
  constexpr int V = 16 / sizeof(T);
  if (hidden % V) return false;
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  return true;
}

}  // namespace
}  // namespace eg

using namespace eg;

// Workspace: nparams x [G, hidden] fp32 partials.
static size_t norm_workspace_bytes(int64_t rows, int64_t hidden, int nparams) {
  if (rows <= 0 || hidden <= 0) return 0;
  const int64_t G = partial_blocks(rows);
  return (size_t)nparams * (size_t)G * (size_t)hidden * sizeof(float);
}

extern "C" size_t eg_rmsnorm_workspace_bytes(int64_t rows, int64_t hidden) {
  return norm_workspace_bytes(rows, hidden, 1);
}

extern "C" size_t eg_layernorm_workspace_bytes(int64_t rows, int64_t hidden) {
  return norm_workspace_bytes(rows, hidden, 2);
}

extern "C" int eg_rmsnorm_fwd(const void* x, const void* weight, void* y, float* rstd,
                              int64_t rows, int64_t hidden, float eps, int dtype,
                              void* stream) {
  clear_error();
  if (check_norm_dims("eg_rmsnorm_fwd", rows, hidden)) return 1;
  if (rows == 0) return 0;
  if (!x || !weight || !y || !rstd) { set_error("eg_rmsnorm_fwd: null pointer"); return 1; }
  hipStream_t st = as_stream(stream);
  return EG_DISPATCH_FLOAT(dtype, "eg_rmsnorm_fwd", [&] {
    using T = scalar_t;
    constexpr int V = 16 / sizeof(T);
    const int h = (int)hidden;
    bool ok;
    const int waves_items = h / (kWave * V);
    if (vec_ok<T>(h, {x, weight, y}) && h % (kWave * V) == 0 &&
        (waves_items == 1 || waves_items == 2 || waves_items == 4 || waves_items == 8)) {
      const unsigned grid = (unsigned)((rows + 3) / 4);
      const T* xp = (const T*)x;
      const T* wp = (const T*)weight;
      T* yp = (T*)y;
      switch (waves_items) {
        case 1: hipLaunchKernelGGL((rmsnorm_fwd_wave<T, V, 1>), dim3(grid), dim3(256), 0, st, xp, wp, yp, rstd, rows, eps); break;
        case 2: hipLaunchKernelGGL((rmsnorm_fwd_wave<T, V, 2>), dim3(grid), dim3(256), 0, st, xp, wp, yp, rstd, rows, eps); break;
        case 4: hipLaunchKernelGGL((rmsnorm_fwd_wave<T, V, 4>), dim3(grid), dim3(256), 0, st, xp, wp, yp, rstd, rows, eps); break;
        default: hipLaunchKernelGGL((rmsnorm_fwd_wave<T, V, 8>), dim3(grid), dim3(256), 0, st, xp, wp, yp, rstd, rows, eps); break;
      }
      ok = true;
    } else if (vec_ok<T>(h, {x, weight, y})) {
      RmsFwd<T, V> f{(const T*)x, (const T*)weight, (T*)y, rstd, rows, h, eps, st};
      ok = pick_norm_config((h + V - 1) / V, f);
    } else {
      RmsFwd<T, 1> f{(const T*)x, (const T*)weight, (T*)y, rstd, rows, h, eps, st};
      ok = pick_norm_config(h, f);
    }
    if (!ok) { set_error("eg_rmsnorm_fwd: hidden=%d too wide", h); return 1; }
    return check_launch("eg_rmsnorm_fwd");
  });
}

extern "C" int eg_rmsnorm_bwd(const void* dy, const void* x, const void* weight,
                              const float* rstd, void* dx, void* dweight, void* workspace,
                              int64_t rows, int64_t hidden, int dtype, void* stream) {
  clear_error();
  if (check_norm_dims("eg_rmsnorm_bwd", rows, hidden)) return 1;
  if (!dweight) { set_error("eg_rmsnorm_bwd: null dweight"); return 1; }
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    // Empty batch: dweight is a sum over no rows.
    size_t es = dtype == EG_F32 ? 4 : 2;
    return zero_fill(dweight, (size_t)hidden * es, st, "eg_rmsnorm_bwd");
  }
  if (!dy || !x || !weight || !rstd || !dx || !workspace) {
    set_error("eg_rmsnorm_bwd: null pointer");
    return 1;
  }
  return EG_DISPATCH_FLOAT(dtype, "eg_rmsnorm_bwd", [&] {
    using T = scalar_t;
    constexpr int V = 16 / sizeof(T);
    const int h = (int)hidden;
    float* part = (float*)workspace;
    bool ok;
    if (vec_ok<T>(h, {dy, x, weight, dx})) {
      RmsBwd<T, V> f{(const T*)dy, (const T*)x, (const T*)weight, rstd, (T*)dx, part, rows, h, st};
      ok = pick_norm_config((h + V - 1) / V, f);
    } else {
      RmsBwd<T, 1> f{(const T*)dy, (const T*)x, (const T*)weight, rstd, (T*)dx, part, rows, h, st};
      ok = pick_norm_config(h, f);
    }
    if (!ok) { set_error("eg_rmsnorm_bwd: hidden=%d too wide", h); return 1; }
    if (int rc = check_launch("eg_rmsnorm_bwd")) return rc;
    const int G = (int)partial_blocks(rows);
    return launch_colsum<T>(part, (T*)dweight, (T*)dweight, 1, G, h, st, "eg_rmsnorm_bwd(colsum)");
  });
}

extern "C" int eg_layernorm_fwd(const void* x, const void* weight, const void* bias, void* y,
                                float* mean, float* rstd, int64_t rows, int64_t hidden,
                                float eps, int dtype, void* stream) {
  clear_error();
  if (check_norm_dims("eg_layernorm_fwd", rows, hidden)) return 1;
  if (rows == 0) return 0;
  if (!x || !weight || !bias || !y || !mean || !rstd) {
    set_error("eg_layernorm_fwd: null pointer");
    return 1;
  }
  hipStream_t st = as_stream(stream);
  return EG_DISPATCH_FLOAT(dtype, "eg_layernorm_fwd", [&] {
    using T = scalar_t;
    constexpr int V = 16 / sizeof(T);
    const int h = (int)hidden;
    bool ok;
    if (vec_ok<T>(h, {x, weight, bias, y})) {
      LnFwd<T, V> f{(const T*)x, (const T*)weight, (const T*)bias, (T*)y, mean, rstd, rows, h, eps, st};
      ok = pick_norm_config((h + V - 1) / V, f);
    } else {
      LnFwd<T, 1> f{(const T*)x, (const T*)weight, (const T*)bias, (T*)y, mean, rstd, rows, h, eps, st};
      ok = pick_norm_config(h, f);
    }
    if (!ok) { set_error("eg_layernorm_fwd: hidden=%d too wide", h); return 1; }
    return check_launch("eg_layernorm_fwd");
  });
}

extern "C" int eg_layernorm_bwd(const void* dy, const void* x, const void* weight,
                                const float* mean, const float* rstd, void* dx, void* dweight,
                                void* dbias, void* workspace, int64_t rows, int64_t hidden,
                                int dtype, void* stream) {
  clear_error();
  if (check_norm_dims("eg_layernorm_bwd", rows, hidden)) return 1;
  if (!dweight || !dbias) { set_error("eg_layernorm_bwd: null dweight/dbias"); return 1; }
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    size_t es = dtype == EG_F32 ? 4 : 2;
    if (int rc = zero_fill(dweight, (size_t)hidden * es, st, "eg_layernorm_bwd")) return rc;
    return zero_fill(dbias, (size_t)hidden * es, st, "eg_layernorm_bwd");
  }
  if (!dy || !x || !weight || !mean || !rstd || !dx || !workspace) {
    set_error("eg_layernorm_bwd: null pointer");
    return 1;
  }
  return EG_DISPATCH_FLOAT(dtype, "eg_layernorm_bwd", [&] {
    using T = scalar_t;
    constexpr int V = 16 / sizeof(T);
    const int h = (int)hidden;
    float* pw = (float*)workspace;
    float* pb = pw + partial_blocks(rows) * (int64_t)h;
    bool ok;
    if (vec_ok<T>(h, {dy, x, weight, dx})) {
      LnBwd<T, V> f{(const T*)dy, (const T*)x, (const T*)weight, mean, rstd, (T*)dx, pw, pb, rows, h, st};
      ok = pick_norm_config((h + V - 1) / V, f);
    } else {
      LnBwd<T, 1> f{(const T*)dy, (const T*)x, (const T*)weight, mean, rstd, (T*)dx, pw, pb, rows, h, st};
      ok = pick_norm_config(h, f);
    }
    if (!ok) { set_error("eg_layernorm_bwd: hidden=%d too wide", h); return 1; }
    if (int rc = check_launch("eg_layernorm_bwd")) return rc;
    const int G = (int)partial_blocks(rows);
    return launch_colsum<T>(pw, (T*)dweight, (T*)dbias, 2, G, h, st, "eg_layernorm_bwd(colsum)");
  });
}
