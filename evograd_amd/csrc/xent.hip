// Hard-label mean cross entropy over vocabulary-wide rows, for gfx950.
//
// Forward restates cross_entropy_forward_ref
// (src/evograd/ops/level1/cross_entropy/forward_ref.py:6-12): per row
// lse = logsumexp(logits[r]) in fp32, the row loss lse - logits[r, target[r]],
// the mean over rows whose target is not ignore_index (-100 in the reference),
// cast to the logits dtype. Backward is the rule of
// src/evograd/ops/level1/cross_entropy/__init__.py:91-94:
// dlogits = dloss * (softmax(logits) - onehot(target)) / n_valid, zero on ignored
// rows.
//
// Saved state is lse [rows] fp32 and n_valid (one fp32 count) beside the inputs.
// Kernels:
//   xent_lse_kernel   one workgroup per row, one HBM read of the row: 16-byte
//                     non-temporal loads, kUnroll packs in flight per thread, an
//                     online (max, sum of exp2) per thread, one max and one sum
//                     over the workgroup; writes lse[row] and the row loss
//                     lse - logits[row, target] (the target logit gathered by
//                     thread 0) into the workspace.
//   xent_mean_kernel  one workgroup: the row losses summed in a fixed order and
//                     the non-ignored rows counted; writes the loss and n_valid.
//   xent_bwd_flat_kernel  wide rows: one read of the logits and one write of
//                     dlogits, workgroups in address order over the flattened
//                     matrix; dloss read from device memory.
//   xent_bwd_rows_kernel  narrow rows: one workgroup per row.
//   scale_copy_kernel dst = src * mul / div with a dtype conversion (the fused
//                     linear cross entropy's dweight conversion and its dloss / n
//                     scaling).
// The fused linear cross entropy (eg_flce_fwd) with fp32 inputs runs
// xent_lse_kernel and the backward kernels on each chunk's fp32 logits, the
// backward with unit scale and a padded output row stride; with 16-bit inputs the
// logits product forms the softmax terms itself and the fix-up (flce_fix_stats_kernel
// and flce_fix_apply_kernel for wide rows, flce_fixup_kernel otherwise) finishes
// each row.
// No atomics: every sum has a fixed order, so results are bitwise repeatable.
//
// A target outside [0, cols) that is not ignore_index makes that row's loss and
// gradient NaN (torch raises there); it is never used as an index.
#include "rowwise.hpp"

namespace eg {
namespace {

using rowwise::kFlatBlock;
using rowwise::kFlatPer;
using rowwise::kFlatUnroll;
using rowwise::kLog2e;
using rowwise::kUnroll;
using rowwise::pick_row_block;
constexpr int kBwdBlock = 256;
constexpr int kMeanBlock = 1024;

template <typename T, int VEC, int BLOCK, bool NT>
__global__ __launch_bounds__(BLOCK) void xent_lse_kernel(const T* __restrict__ x,
                                                         const int64_t* __restrict__ target,
                                                         float* __restrict__ lse,
                                                         float* __restrict__ rowloss, int cols,
                                                         int64_t ignore_index) {
  __shared__ float red[BLOCK / kWave];
  const int64_t row = blockIdx.x;
  const T* __restrict__ xr = x + row * cols;
  // The target logit is gathered before the row stream starts, so its latency
  // overlaps the first batch of loads.
  int64_t t = 0;
  float picked = 0.f;
  if (threadIdx.x == 0) {
    t = target[row];
    if (t != ignore_index) picked = (t >= 0 && t < cols) ? to_f32(xr[t]) : NAN;
  }
  const float l = rowwise::row_lse<T, VEC, BLOCK, NT>(xr, cols, red);
  if (threadIdx.x == 0) {
    lse[row] = l;
    rowloss[row] = (t == ignore_index) ? 0.f : l - picked;
  }
}

// One workgroup; each thread takes kMeanRows rows per pass with all their loads
// issued before any is used, then a fixed-order workgroup sum.
constexpr int kMeanRows = 8;

template <typename T>
__global__ __launch_bounds__(kMeanBlock) void xent_mean_kernel(
    const int64_t* __restrict__ target, const float* __restrict__ rowloss, T* __restrict__ loss,
    float* __restrict__ n_valid, int64_t rows, int64_t ignore_index) {
  __shared__ float red[kMeanBlock / kWave];
  float sum = 0.f, count = 0.f;
  for (int64_t r0 = threadIdx.x; r0 < rows; r0 += (int64_t)kMeanBlock * kMeanRows) {
    float l[kMeanRows], ok[kMeanRows];
#pragma unroll
    for (int j = 0; j < kMeanRows; ++j) {
      const int64_t r = r0 + (int64_t)j * kMeanBlock;
      const bool in = r < rows;
      ok[j] = (in && target[r] != ignore_index) ? 1.f : 0.f;
      l[j] = in ? rowloss[r] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < kMeanRows; ++j) {
      sum += l[j];
      count += ok[j];
    }
  }
  sum = block_reduce<kMeanBlock>(sum, SumOp(), red);
  count = block_reduce<kMeanBlock>(count, SumOp(), red);
  if (threadIdx.x == 0) {
    loss[0] = from_f32<T>(sum / count);
    n_valid[0] = count;
  }
}

// Per-row factors of the backward: g = dloss / n_valid, or 1 when dloss is null
// (the unit gradient softmax - onehot of the fused linear cross entropy); NaN
// for an out-of-range target. Also lse in log2 units, the target column, and
// whether the row is ignored.
struct RowGrad {
  float g, ll;
  int tc;
  bool ignored;
};

template <typename TD>
__device__ __forceinline__ RowGrad row_grad(const TD* __restrict__ dloss,
                                            const int64_t* __restrict__ target,
                                            const float* __restrict__ lse,
                                            const float* __restrict__ n_valid, int64_t row,
                                            int cols, int64_t ignore_index) {
  const int64_t t = target[row];
  RowGrad r;
  r.ignored = t == ignore_index;
  const float g = dloss ? to_f32(dloss[0]) / n_valid[0] : 1.f;
  r.g = (t >= 0 && t < cols) ? g : NAN;
  r.ll = lse[row] * kLog2e;
  r.tc = (int)t;
  return r;
}

// dlogits of one pack of VEC columns starting at column c of a row.
template <int VEC>
__device__ __forceinline__ void grad_pack(const RowGrad& rg, int c, const float (&v)[VEC],
                                          float (&o)[VEC]) {
  if (rg.ignored) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) o[i] = 0.f;
    return;
  }
#pragma unroll
  for (int i = 0; i < VEC; ++i)
    o[i] = rg.g * __builtin_amdgcn_exp2f(__builtin_fmaf(v[i], kLog2e, -rg.ll));
  const unsigned k = (unsigned)(rg.tc - c);
  if (k < (unsigned)VEC) {
    // the target column: g * (p - 1)
#pragma unroll
    for (int i = 0; i < VEC; ++i)
      if (i == (int)k) o[i] -= rg.g;
  }
}

// Wide rows: the matrix as one flat sequence of packs, workgroup b covering
// packs [b * kFlatPer, (b + 1) * kFlatPer) in address order, so the workgroups in
// flight stream through contiguous memory. A workgroup spans at most two rows
// (packs per row >= kFlatPer, checked by the host). TI is the logits type, TO the
// gradient's, TD the type of dloss.
template <typename TI, typename TO, typename TD, int VEC, bool NT>
__global__ __launch_bounds__(kFlatBlock) void xent_bwd_flat_kernel(
    const TD* __restrict__ dloss, const TI* __restrict__ x, const int64_t* __restrict__ target,
    const float* __restrict__ lse, const float* __restrict__ n_valid, TO* __restrict__ dx,
    int64_t rows, int cols, int64_t ldd, int64_t ignore_index) {
  const int64_t ppr = cols / VEC;  // packs per row
  const int64_t npack = rows * ppr;
  const int64_t first = (int64_t)blockIdx.x * kFlatPer;
  const int64_t row0 = first / ppr;
  const int64_t bound = (row0 + 1) * ppr;  // first pack of the next row
  const RowGrad r0 = row_grad(dloss, target, lse, n_valid, row0, cols, ignore_index);
  const bool two = first + kFlatPer > bound && row0 + 1 < rows;
  const RowGrad r1 = two ? row_grad(dloss, target, lse, n_valid, row0 + 1, cols, ignore_index)
                         : r0;
  float v[kFlatUnroll][VEC];
#pragma unroll
  for (int u = 0; u < kFlatUnroll; ++u) {
    const int64_t p = first + u * kFlatBlock + threadIdx.x;
    if (p < npack) load_vec<TI, VEC, NT>(x + p * VEC, v[u]);
  }
#pragma unroll
  for (int u = 0; u < kFlatUnroll; ++u) {
    const int64_t p = first + u * kFlatBlock + threadIdx.x;
    if (p < npack) {
      const bool hi = p >= bound;
      const int c = (int)((hi ? p - bound : p - row0 * ppr) * VEC);
      float o[VEC];
      grad_pack<VEC>(hi ? r1 : r0, c, v[u], o);
      store_vec<TO, VEC, NT>(dx + (row0 + (hi ? 1 : 0)) * ldd + c, o);
    }
  }
}

// Narrow rows (fewer packs than one flat workgroup covers): one workgroup per row.
template <typename TI, typename TO, typename TD, int VEC, bool NT>
__global__ __launch_bounds__(kBwdBlock) void xent_bwd_rows_kernel(
    const TD* __restrict__ dloss, const TI* __restrict__ x, const int64_t* __restrict__ target,
    const float* __restrict__ lse, const float* __restrict__ n_valid, TO* __restrict__ dx,
    int cols, int64_t ldd, int64_t ignore_index) {
  constexpr int STEP = kBwdBlock * VEC;
  const int64_t row = blockIdx.x;
  const RowGrad rg = row_grad(dloss, target, lse, n_valid, row, cols, ignore_index);
  const int c0 = (int)blockIdx.y * (STEP * kUnroll) + (int)threadIdx.x * VEC;
  const TI* __restrict__ xr = x + row * cols;
  TO* __restrict__ dr = dx + row * ldd;
  float v[kUnroll][VEC];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int c = c0 + u * STEP;
    if (c < cols && !rg.ignored) load_vec<TI, VEC, NT>(xr + c, v[u]);
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int c = c0 + u * STEP;
    if (c < cols) {
      float o[VEC];
      grad_pack<VEC>(rg, c, v[u], o);
      store_vec<TO, VEC, NT>(dr + c, o);
    }
  }
}

// dst[i] = src[i] * mul[0] / div[0] (either factor optional). Workgroups cover
// consecutive runs of kScaleUnroll x 256 packs in address order, every load of a
// thread issued before its first store.
constexpr int kScaleUnroll = 4;

template <typename TS, typename TO, typename TM, int VEC>
__global__ __launch_bounds__(256) void scale_copy_kernel(const TS* __restrict__ src,
                                                         TO* __restrict__ dst, int64_t npack,
                                                         const TM* __restrict__ mul,
                                                         const float* __restrict__ div) {
  // A zero divisor (no row counted toward a mean loss) scales by 0: the unit
  // gradients are all zero then, and torch's gradient of such a loss is zero too.
  const float d = div ? div[0] : 1.f;
  const float f = d != 0.f ? (mul ? to_f32(mul[0]) : 1.f) / d : 0.f;
  const int64_t p0 = (int64_t)blockIdx.x * (256 * kScaleUnroll) + threadIdx.x;
  float v[kScaleUnroll][VEC];
#pragma unroll
  for (int u = 0; u < kScaleUnroll; ++u) {
    const int64_t p = p0 + u * 256;
    if (p < npack) load_vec<TS, VEC, VEC * sizeof(TS) == 16>(src + p * VEC, v[u]);
  }
#pragma unroll
  for (int u = 0; u < kScaleUnroll; ++u) {
    const int64_t p = p0 + u * 256;
    if (p < npack) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) v[u][i] *= f;
      store_vec<TO, VEC, VEC * sizeof(TO) == 16>(dst + p * VEC, v[u]);
    }
  }
}

template <typename T, int VEC>
struct LseLaunch {
  const T* x; const int64_t* target; float* lse; float* rowloss; int64_t rows; int cols;
  int64_t ignore_index; hipStream_t st;
  template <int BLOCK> void go() {
    EG_LAUNCH((xent_lse_kernel<T, VEC, BLOCK, VEC * sizeof(T) == 16>), dim3((unsigned)rows),
              dim3(BLOCK), 0, st, x, target, lse, rowloss, cols, ignore_index);
  }
};

template <typename TI, typename TO, typename TD, int VEC>
// dlogits rows are written with row stride ldd (>= cols, a multiple of VEC).
void launch_bwd(const TD* gp, const TI* xp, const int64_t* target, const float* lse,
                const float* n_valid, TO* dp, int64_t rows, int cols, int64_t ignore_index,
                hipStream_t st, int64_t ldd = -1) {
  constexpr bool NT = VEC * sizeof(TI) == 16;
  if (ldd < 0) ldd = cols;
  const int64_t ppr = cols / VEC;
  if (ppr >= kFlatPer) {
    const int64_t blocks = (rows * ppr + kFlatPer - 1) / kFlatPer;
    EG_LAUNCH((xent_bwd_flat_kernel<TI, TO, TD, VEC, NT>), dim3((unsigned)blocks),
              dim3(kFlatBlock), 0, st, gp, xp, target, lse, n_valid, dp, rows, cols, ldd,
              ignore_index);
  } else {
    EG_LAUNCH((xent_bwd_rows_kernel<TI, TO, TD, VEC, NT>), dim3((unsigned)rows, 1u),
              dim3(kBwdBlock), 0, st, gp, xp, target, lse, n_valid, dp, cols, ldd,
              ignore_index);
  }
}

int check_xent(const char* what, int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) {
    set_error("%s: negative size rows=%lld cols=%lld", what, (long long)rows, (long long)cols);
    return 1;
  }
  if (rows > 0 && cols == 0) {
    set_error("%s: cross entropy over zero classes", what);
    return 1;
  }
  // rows: the grid's x extent and an exactly representable fp32 count; cols: int.
  if (rows > ((int64_t)1 << 24) || cols > ((int64_t)1 << 30)) {
    set_error("%s: size out of range rows=%lld cols=%lld", what, (long long)rows,
              (long long)cols);
    return 1;
  }
  return 0;
}

}  // namespace
}  // namespace eg

using namespace eg;

extern "C" size_t eg_cross_entropy_workspace_bytes(int64_t rows) {
  return rows > 0 ? (size_t)rows * sizeof(float) : 0;
}

extern "C" int eg_cross_entropy_fwd(const void* logits, const int64_t* target, void* loss,
                                    float* lse, float* n_valid, void* workspace, int64_t rows,
                                    int64_t cols, int64_t ignore_index, int dtype,
                                    void* stream) {
  clear_error();
  if (check_xent("eg_cross_entropy_fwd", rows, cols)) return 1;
  if (!loss || !n_valid || (rows > 0 && (!logits || !target || !lse || !workspace))) {
    set_error("eg_cross_entropy_fwd: null pointer");
    return 1;
  }
  hipStream_t st = as_stream(stream);
  float* rowloss = static_cast<float*>(workspace);
  return EG_DISPATCH_FLOAT(dtype, "eg_cross_entropy_fwd", [&] {
    using T = scalar_t;
    constexpr int V = 16 / sizeof(T);
    const T* xp = static_cast<const T*>(logits);
    if (rows > 0) {
      if (cols % V == 0 && aligned16(logits)) {
        pick_row_block(cols / V, LseLaunch<T, V>{xp, target, lse, rowloss, rows, (int)cols,
                                                 ignore_index, st});
      } else {
        pick_row_block(cols, LseLaunch<T, 1>{xp, target, lse, rowloss, rows, (int)cols,
                                             ignore_index, st});
      }
    }
    // Also for rows == 0: the mean of no rows is 0/0 (NaN), as in torch.
    EG_LAUNCH((xent_mean_kernel<T>), dim3(1), dim3(kMeanBlock), 0, st, target, rowloss,
              static_cast<T*>(loss), n_valid, rows, ignore_index);
    return check_launch("eg_cross_entropy_fwd");
  });
}

extern "C" int eg_cross_entropy_bwd(const void* dloss, const void* logits,
                                    const int64_t* target, const float* lse,
                                    const float* n_valid, void* dlogits, int64_t rows,
                                    int64_t cols, int64_t ignore_index, int dtype,
                                    void* stream) {
  clear_error();
  if (check_xent("eg_cross_entropy_bwd", rows, cols)) return 1;
  if (rows == 0) return 0;
  if (!dloss || !logits || !target || !lse || !n_valid || !dlogits) {
    set_error("eg_cross_entropy_bwd: null pointer");
    return 1;
  }
  // flat grid: at most 2^32 threads in x
  if (rows * cols / kFlatPer >= ((int64_t)1 << 32) / kFlatBlock) {
    set_error("eg_cross_entropy_bwd: rows*cols=%lld exceeds the launch grid",
              (long long)(rows * cols));
    return 1;
  }
  hipStream_t st = as_stream(stream);
  return EG_DISPATCH_FLOAT(dtype, "eg_cross_entropy_bwd", [&] {
    using T = scalar_t;
    constexpr int V = 16 / sizeof(T);
    const T* gp = static_cast<const T*>(dloss);
    const T* xp = static_cast<const T*>(logits);
    T* dp = static_cast<T*>(dlogits);
    if (cols % V == 0 && aligned16(logits) && aligned16(dlogits))
      launch_bwd<T, T, T, V>(gp, xp, target, lse, n_valid, dp, rows, (int)cols, ignore_index,
                             st);
    else
      launch_bwd<T, T, T, 1>(gp, xp, target, lse, n_valid, dp, rows, (int)cols, ignore_index,
                             st);
    return check_launch("eg_cross_entropy_bwd");
  });
}

// ------------------------------------------------ fused linear cross entropy
// fused_linear_cross_entropy (src/evograd/ops/level2/fused_linear_cross_entropy/
// forward_ref.py:23-35; gradients declared at fused_linear_cross_entropy/
// __init__.py:91-152) in one launch sequence. The gradient is formed in the
// forward (the backward only receives the scalar dloss): per row chunk,
//   16-bit inputs: the logits product x_c W^T (MFMA, gemm_kernel.hpp) with the softmax
//   epilogue writes exp(logit - group max) into the dlogits rows, the group
//   statistics and the target logits -> the fix-up forms lse, the row
//   losses and unit dlogits = softmax - onehot in place (one chunk of all rows by
//   default: no fp32 logits are held);
//   fp32 inputs: logits = x_c W^T (fp32) -> lse and row losses (xent_lse_kernel)
//   -> unit dlogits (xent_bwd_*_kernel), chunks of at most 2^29 logits;
// then dx_c = dl_c W and dW (+)= dl_c^T x_c (MFMA; with more than one chunk the
// products accumulate in an fp32 [vocab, hidden] buffer, added in each product's
// epilogue, and the last chunk's product rounds the sum once into dW; fp32 inputs
// accumulate in dW itself), and the mean loss. Only one chunk of dlogits exists
// at a time (at most kFlceDlChunkBytes by default), so scratch grows with the chunk
// and the vocabulary, not with rows x vocab; dlogits rows are padded to a multiple
// of 64 columns with zeros, the product's k step. No atomics: bitwise repeatable.

namespace eg {
namespace {

template <typename F>
int dispatch_type(int dtype, const char* what, F&& f) {
  switch (dtype) {
    case EG_F32: return f(float{});
    case EG_F16: return f(f16_t{});
    case EG_BF16: return f(bf16_t{});
    default: set_error("%s: unsupported dtype %d", what, dtype); return 1;
  }
}

// Zeroes columns [c0, c1) of every row of a [rows][ld] 16-bit matrix (the padding
// of the dlogits rows).
__global__ __launch_bounds__(256) void zero_cols_kernel(uint16_t* __restrict__ p, int64_t rows,
                                                        int c0, int c1, int64_t ld) {
  const int w = c1 - c0;
  const int64_t n = rows * w;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[(i / w) * ld + c0 + i % w] = 0;
}

// Default chunking: the dlogits of one chunk take at most this many bytes (the
// fp32 path holds as many bytes again of fp32 logits).
constexpr int64_t kFlceDlChunkBytes = (int64_t)1 << 30;

// 16-bit path: the logits product leaves, per 128-column group h of each row,
// e = exp(logit - mx_h) in the dlogits rows, (mx_h, s_h = sum of e) and the target
// logit (gemm_logits_softmax_launch). One workgroup per row then forms
//   lse = M + log(sum_h s_h exp(mx_h - M)),  M = max_h mx_h (0 when infinite),
//   rowloss = lse - logit[target] (0 on an ignored row, NaN for a target outside
//   [0, cols)),
//   dlogits = e * exp(mx_h - lse) - onehot(target) in place (zero on an ignored
//   row, NaN for a bad target),
// one read and one write of the 16-bit rows. The group factors exp(mx_h - lse)
// sit in LDS, so a row holds at most kFixMaxGroups groups.
constexpr int kFixBlock = 1024;
constexpr int kFixUnroll = 4;
constexpr int kFixMaxGroups = 8192;

template <typename T>
__global__ __launch_bounds__(kFixBlock) void flce_fixup_kernel(
    T* __restrict__ e, int64_t lde, int cols, const float* __restrict__ hstats, int nh2,
    const float* __restrict__ tlogit, const int64_t* __restrict__ target,
    float* __restrict__ lse_out, float* __restrict__ rowloss, int64_t ignore_index) {
  __shared__ float fac[kFixMaxGroups];
  __shared__ float red[kFixBlock / kWave];
  const int64_t row = blockIdx.x;
  const int nh = (cols + 127) / 128;
  const float* hs = hstats + row * (int64_t)nh2 * 2;
  float m = -INFINITY;
  for (int h = threadIdx.x; h < nh; h += kFixBlock) m = fmaxf(m, hs[2 * h]);
  m = rowwise::lse_ref(block_reduce<kFixBlock>(m, MaxOp(), red));
  float s = 0.f;
  for (int h = threadIdx.x; h < nh; h += kFixBlock)
    s += hs[2 * h + 1] * __builtin_amdgcn_exp2f((hs[2 * h] - m) * kLog2e);
  s = block_reduce<kFixBlock>(s, SumOp(), red);
  const float lse = m + logf(s);
  const int64_t t = target[row];
  const bool ignored = t == ignore_index;
  const bool bad = !ignored && (t < 0 || t >= cols);
  for (int h = threadIdx.x; h < nh; h += kFixBlock)
    fac[h] = bad ? NAN : __builtin_amdgcn_exp2f((hs[2 * h] - lse) * kLog2e);
  if (threadIdx.x == 0) {
    lse_out[row] = lse;
    rowloss[row] = ignored ? 0.f : (bad ? NAN : lse - tlogit[row]);
  }
  __syncthreads();
  T* er = e + row * lde;
  const int tc = bad || ignored ? -1 : (int)t;
  // packs of 8 columns (8 divides 128: one group per pack)
  const int np = cols / 8;
  for (int p0 = threadIdx.x; p0 < np; p0 += kFixBlock * kFixUnroll) {
    float v[kFixUnroll][8];
#pragma unroll
    for (int u = 0; u < kFixUnroll; ++u) {
      const int p = p0 + u * kFixBlock;
      if (p < np) load_vec<T, 8, true>(er + 8 * p, v[u]);
    }
#pragma unroll
    for (int u = 0; u < kFixUnroll; ++u) {
      const int p = p0 + u * kFixBlock;
      if (p < np) {
        const float f = fac[p >> 4];
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = ignored ? 0.f : v[u][i] * f;
        const unsigned k = (unsigned)(tc - 8 * p);
        if (k < 8u) {
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (i == (int)k) o[i] -= 1.f;
        }
        store_vec<T, 8, true>(er + 8 * p, o);
      }
    }
  }
  for (int c = np * 8 + threadIdx.x; c < cols; c += kFixBlock) {
    float o = ignored ? 0.f : to_f32(er[c]) * fac[c >> 7];
    if (c == tc) o -= 1.f;
    er[c] = from_f32<T>(o);
  }
}

// Rows of whole 8-column packs with at least kFlatPer packs and at most
// kStatBlock * kStatPer groups: the same fix-up in two launches.
// flce_fix_stats_kernel, one 256-thread workgroup per row, loads all of the row's
// group statistics at once (kStatPer groups per thread, in registers), forms lse
// and the row loss, and writes the group factors exp(mx_h - lse) into the first
// nh floats of the row's statistics (every read of the row is behind the
// reductions' barriers). flce_fix_apply_kernel then takes the chunk's dlogits as one
// flat sequence of packs, workgroup b covering packs [b * kFlatPer, (b + 1) *
// kFlatPer) in address order (at most two rows), so the workgroups in flight
// stream through contiguous memory (bf16 [4096, 128256], e written just before:
// 353 us against 388 us for the loop over each row and 372 us for the row held in
// registers; the factors take 13 us, 36 us with a 1024-thread workgroup per row).
constexpr int kStatBlock = 256, kStatPer = 4;

__global__ __launch_bounds__(kStatBlock) void flce_fix_stats_kernel(
    int cols, float* __restrict__ hstats, int nh2, const float* __restrict__ tlogit,
    const int64_t* __restrict__ target, float* __restrict__ lse_out,
    float* __restrict__ rowloss, int64_t ignore_index) {
  __shared__ float red[kStatBlock / kWave];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nh = (cols + 127) / 128;
  float* hs = hstats + row * (int64_t)nh2 * 2;
  float2 g[kStatPer];
#pragma unroll
  for (int j = 0; j < kStatPer; ++j) {
    const int h = j * kStatBlock + tid;
    g[j] = h < nh ? *reinterpret_cast<const float2*>(hs + 2 * h) : make_float2(-INFINITY, 0.f);
  }
  float m = g[0].x;
#pragma unroll
  for (int j = 1; j < kStatPer; ++j) m = fmaxf(m, g[j].x);
  m = rowwise::lse_ref(block_reduce<kStatBlock>(m, MaxOp(), red));
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kStatPer; ++j)
    if (j * kStatBlock + tid < nh) s += g[j].y * __builtin_amdgcn_exp2f((g[j].x - m) * kLog2e);
  s = block_reduce<kStatBlock>(s, SumOp(), red);
  const float lse = m + logf(s);
  const int64_t t = target[row];
  const bool ignored = t == ignore_index;
  const bool bad = !ignored && (t < 0 || t >= cols);
#pragma unroll
  for (int j = 0; j < kStatPer; ++j) {
    const int h = j * kStatBlock + tid;
    if (h < nh) hs[h] = bad ? NAN : __builtin_amdgcn_exp2f((g[j].x - lse) * kLog2e);
  }
  if (tid == 0) {
    lse_out[row] = lse;
    rowloss[row] = ignored ? 0.f : (bad ? NAN : lse - tlogit[row]);
  }
}

template <typename T>
__global__ __launch_bounds__(kFlatBlock) void flce_fix_apply_kernel(
    T* __restrict__ e, int64_t lde, int64_t rows, int cols, const float* __restrict__ hstats,
    int nh2, const int64_t* __restrict__ target, int64_t ignore_index) {
  const int64_t ppr = cols / 8;  // packs per row
  const int64_t npack = rows * ppr;
  const int64_t first = (int64_t)blockIdx.x * kFlatPer;
  const int64_t row0 = first / ppr;
  const int64_t bound = (row0 + 1) * ppr;  // first pack of the next row
  // per row: the target column (-1 for none) and whether the row is ignored
  auto tcol = [&](int64_t r, bool& ign) {
    const int64_t t = target[r];
    ign = t == ignore_index;
    return ign || t < 0 || t >= cols ? -1 : (int)t;
  };
  bool ign0 = false, ign1 = false;
  const int tc0 = tcol(row0, ign0);
  const int tc1 = row0 + 1 < rows ? tcol(row0 + 1, ign1) : -1;
  float v[kFlatUnroll][8];
#pragma unroll
  for (int u = 0; u < kFlatUnroll; ++u) {
    const int64_t p = first + u * kFlatBlock + threadIdx.x;
    if (p < npack) {
      const bool hi = p >= bound;
      const int64_t pc = hi ? p - bound : p - row0 * ppr;
      load_vec<T, 8, true>(e + (row0 + (hi ? 1 : 0)) * lde + 8 * pc, v[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kFlatUnroll; ++u) {
    const int64_t p = first + u * kFlatBlock + threadIdx.x;
    if (p < npack) {
      const bool hi = p >= bound;
      const int64_t r = row0 + (hi ? 1 : 0);
      const int pc = (int)(hi ? p - bound : p - row0 * ppr);
      const float f = hstats[r * nh2 * 2 + (pc >> 4)];  // the pack's group factor
      const bool ign = hi ? ign1 : ign0;
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = ign ? 0.f : v[u][i] * f;
      const unsigned k = (unsigned)((hi ? tc1 : tc0) - 8 * pc);
      if (k < 8u) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (i == (int)k) o[i] -= 1.f;
      }
      store_vec<T, 8, true>(e + r * lde + 8 * pc, o);
    }
  }
}

// Rows per chunk by default: as many as kFlceDlChunkBytes of dlogits rows allow
// (row_bytes each), all rows when they fit, else a multiple of 256 (the product's
// row tile) or, below that, a power of two.
int64_t flce_chunk_rows(int64_t rows, int64_t row_bytes) {
  int64_t rc = kFlceDlChunkBytes / (row_bytes > 0 ? row_bytes : 1);
  if (rc < 1) rc = 1;
  if (rc >= rows) return rows > 0 ? rows : 1;
  if (rc >= 256) return rc / 256 * 256;
  int64_t p = 1;
  while (p * 2 <= rc) p *= 2;
  return p;
}

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Whether the 16-bit path (softmax terms formed in the logits product's epilogue)
// takes this call; fp32 inputs, and rows of more than kFixMaxGroups groups, keep fp32
// logits chunks.
bool flce_fused(int64_t vocab, int dtype) {
  return dtype != EG_F32 && (vocab + 127) / 128 <= kFixMaxGroups;
}

// Workspace: [lse | rowloss] (fp32, rows each), then either one chunk of fp32 logits
// or (16-bit path) the target logits [rows] and the group statistics of one chunk
// [rc][flce_groups(vocab)][2], then the dlogits of one chunk [rc][vp], then (16-bit
// inputs over more than one chunk) the fp32 dW sum [vocab][hidden].
struct FlceLayout {
  int64_t rc, vp;
  bool fused;
  size_t stats, logits, dl, acc, total;
};

FlceLayout flce_layout(int64_t rows, int64_t hidden, int64_t vocab, int64_t chunk_rows,
                       int dtype) {
  FlceLayout l;
  l.fused = flce_fused(vocab, dtype);
  const int64_t all = rows > 0 ? rows : 1;
  l.vp = dtype == EG_F32 ? vocab : (vocab + 63) / 64 * 64;
  const size_t es = dtype == EG_F32 ? 4 : 2;
  l.rc = chunk_rows > 0 ? std::min(chunk_rows, all) : flce_chunk_rows(rows, l.vp * (int64_t)es);
  l.stats = align_up((size_t)rows * 2 * sizeof(float));
  l.logits = l.fused ? align_up((size_t)rows * sizeof(float)) +
                           align_up((size_t)l.rc * flce_groups(vocab) * 2 * sizeof(float))
                     : align_up((size_t)l.rc * vocab * sizeof(float));
  l.dl = align_up((size_t)l.rc * l.vp * es);
  l.acc = (dtype != EG_F32 && rows > l.rc) ? align_up((size_t)vocab * hidden * sizeof(float)) : 0;
  l.total = l.stats + l.logits + l.dl + l.acc;
  return l;
}

}  // namespace
}  // namespace eg

extern "C" size_t eg_flce_workspace_bytes(int64_t rows, int64_t hidden, int64_t vocab,
                                          int64_t chunk_rows, int dtype) {
  if (rows <= 0 || vocab <= 0) return 0;
  return flce_layout(rows, hidden, vocab, chunk_rows, dtype).total;
}

extern "C" int eg_flce_fwd(const void* x, const void* weight, const int64_t* target, float* loss,
                           void* dx, void* dweight, float* n_valid, void* workspace,
                           int64_t rows, int64_t hidden, int64_t vocab, int64_t ignore_index,
                           int64_t chunk_rows, int dtype, void* stream) {
  static const char* name = "eg_flce_fwd";
  clear_error();
  if (check_xent(name, rows, vocab)) return 1;
  if (hidden <= 0 || hidden > ((int64_t)1 << 20)) {
    set_error("%s: hidden=%lld out of range", name, (long long)hidden);
    return 1;
  }
  if (dtype != EG_F32 && dtype != EG_F16 && dtype != EG_BF16) {
    set_error("%s: unsupported dtype %d", name, dtype);
    return 1;
  }
  if (dtype != EG_F32 && hidden % 64) {
    set_error("%s: 16-bit inputs need hidden %% 64 == 0 (pad x and weight with zero columns)",
              name);
    return 1;
  }
  if (!loss || !n_valid || !dweight || (rows > 0 && (!x || !weight || !target || !dx ||
                                                     !workspace))) {
    set_error("%s: null pointer", name);
    return 1;
  }
  if (!aligned16(x) || !aligned16(weight) || !aligned16(workspace)) {
    set_error("%s: x, weight and workspace must be 16-byte aligned", name);
    return 1;
  }
  const FlceLayout L = flce_layout(rows, hidden, vocab, chunk_rows, dtype);
  if (L.rc * vocab / kFlatPer >= ((int64_t)1 << 32) / kFlatBlock) {
    set_error("%s: vocab=%lld exceeds the launch grid", name, (long long)vocab);
    return 1;
  }
  hipStream_t st = as_stream(stream);
  const size_t es = dtype == EG_F32 ? 4 : 2;
  if (rows == 0) {
    // no rows: dweight is a sum over nothing; the mean loss is 0 / 0
    if (int rc = zero_fill(dweight, (size_t)vocab * hidden * es, st, name)) return rc;
    EG_LAUNCH((xent_mean_kernel<float>), dim3(1), dim3(kMeanBlock), 0, st, target, nullptr,
              loss, n_valid, rows, ignore_index);
    return check_launch(name);
  }
  char* ws = (char*)workspace;
  float* lse = (float*)ws;
  float* rowloss = lse + rows;
  float* logits = (float*)(ws + L.stats);
  char* dl = ws + L.stats + L.logits;
  float* acc = L.acc ? (float*)(dl + L.dl) : nullptr;
  return dispatch_type(dtype, name, [&](auto tag) {
    using T = decltype(tag);
    T* dlp = (T*)dl;
    if (L.vp > vocab) {
      // padding columns of the chunk's dlogits rows: zero once, never written after
      const int64_t n = L.rc * (L.vp - vocab);
      const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 4096);
      EG_LAUNCH(zero_cols_kernel, dim3(grid), dim3(256), 0, st, (uint16_t*)dl, L.rc, (int)vocab,
                (int)L.vp, L.vp);
    }
    for (int64_t r0 = 0; r0 < rows; r0 += L.rc) {
      const int64_t n = std::min(L.rc, rows - r0);
      const T* xc = (const T*)x + r0 * hidden;
      if (L.fused) {
        float* tlogit = logits;
        float* hstats = (float*)((char*)logits + align_up((size_t)rows * sizeof(float)));
        if (int rc = gemm_logits_softmax_launch(xc, weight, dlp, n, vocab, hidden, hidden, hidden,
                                                L.vp, target + r0, hstats, tlogit + r0, dtype, st,
                                                name))
          return rc;
        if constexpr (!std::is_same<T, float>::value) {
          const int nh2 = (int)flce_groups(vocab);
          if (vocab % 8 == 0 && vocab / 8 >= kFlatPer &&
              (vocab + 127) / 128 <= kStatBlock * kStatPer) {
            // wide rows of whole packs: factors per row, then one flat pass
            EG_LAUNCH(flce_fix_stats_kernel, dim3((unsigned)n), dim3(kStatBlock), 0, st,
                      (int)vocab, hstats, nh2, tlogit + r0, target + r0, lse + r0,
                      rowloss + r0, ignore_index);
            const int64_t blocks = (n * (vocab / 8) + kFlatPer - 1) / kFlatPer;
            EG_LAUNCH((flce_fix_apply_kernel<T>), dim3((unsigned)blocks), dim3(kFlatBlock), 0,
                      st, dlp, L.vp, n, (int)vocab, hstats, nh2, target + r0, ignore_index);
          } else
            EG_LAUNCH((flce_fixup_kernel<T>), dim3((unsigned)n), dim3(kFixBlock), 0, st, dlp,
                      L.vp, (int)vocab, hstats, nh2, tlogit + r0, target + r0, lse + r0,
                      rowloss + r0, ignore_index);
        }
        if (int rc = check_launch(name)) return rc;
      } else {
        if (int rc = gemm_launch(xc, weight, logits, n, vocab, hidden, hidden, hidden, vocab, true,
                                 true, n, vocab, dtype, EG_F32, st, name))
          return rc;
        const float* none = nullptr;
        if (vocab % 4 == 0) {
          pick_row_block(vocab / 4, LseLaunch<float, 4>{logits, target + r0, lse + r0,
                                                        rowloss + r0, n, (int)vocab,
                                                        ignore_index, st});
          launch_bwd<float, T, float, 4>(none, logits, target + r0, lse + r0, nullptr, dlp, n,
                                         (int)vocab, ignore_index, st, L.vp);
        } else {
          pick_row_block(vocab, LseLaunch<float, 1>{logits, target + r0, lse + r0, rowloss + r0,
                                                    n, (int)vocab, ignore_index, st});
          launch_bwd<float, T, float, 1>(none, logits, target + r0, lse + r0, nullptr, dlp, n,
                                         (int)vocab, ignore_index, st, L.vp);
        }
        if (int rc = check_launch(name)) return rc;
      }
      if (int rc = gemm_launch(dlp, weight, (T*)dx + r0 * hidden, n, hidden, L.vp, L.vp, hidden,
                               hidden, true, false, n, vocab, dtype, dtype, st, name))
        return rc;
      // dW = sum over chunks of dl_c^T x_c: into dW directly (one chunk, or fp32
      // inputs), else into the fp32 sum, the last chunk rounding it once into dW
      const bool first = r0 == 0, last = r0 + n >= rows;
      void* out = (acc && !last) ? (void*)acc : dweight;
      const void* res = first ? nullptr : (acc ? (const void*)acc : dweight);
      if (int rc = gemm_launch(dlp, xc, out, vocab, hidden, n, L.vp, hidden, hidden, false,
                               false, n, n, dtype, out == acc ? EG_F32 : dtype, st, name, res,
                               hidden, acc != nullptr))
        return rc;
    }
    EG_LAUNCH((xent_mean_kernel<float>), dim3(1), dim3(kMeanBlock), 0, st, target, rowloss, loss,
              n_valid, rows, ignore_index);
    return check_launch(name);
  });
}

extern "C" int eg_cross_entropy_mean(const int64_t* target, const float* rowloss, void* loss,
                                     float* n_valid, int64_t rows, int64_t ignore_index,
                                     int loss_dtype, void* stream) {
  clear_error();
  if (rows < 0 || rows > ((int64_t)1 << 24)) {
    set_error("eg_cross_entropy_mean: rows=%lld out of range", (long long)rows);
    return 1;
  }
  if (!loss || !n_valid || (rows > 0 && (!target || !rowloss))) {
    set_error("eg_cross_entropy_mean: null pointer");
    return 1;
  }
  hipStream_t st = as_stream(stream);
  return dispatch_type(loss_dtype, "eg_cross_entropy_mean", [&](auto tag) {
    using T = decltype(tag);
    EG_LAUNCH((xent_mean_kernel<T>), dim3(1), dim3(kMeanBlock), 0, st, target, rowloss,
              static_cast<T*>(loss), n_valid, rows, ignore_index);
    return check_launch("eg_cross_entropy_mean");
  });
}

extern "C" int eg_scale_copy(const void* src, int src_dtype, void* dst, int dst_dtype,
                             int64_t n, const void* mul, int mul_dtype, const float* div,
                             void* stream) {
  clear_error();
  if (n < 0) {
    set_error("eg_scale_copy: negative size %lld", (long long)n);
    return 1;
  }
  if (n == 0) return 0;
  if (!src || !dst) {
    set_error("eg_scale_copy: null pointer");
    return 1;
  }
  if (n / (256 * kScaleUnroll) >= 0x7fffffffLL) {
    set_error("eg_scale_copy: n=%lld exceeds the launch grid", (long long)n);
    return 1;
  }
  hipStream_t st = as_stream(stream);
  return dispatch_type(src_dtype, "eg_scale_copy", [&](auto stag) {
    using TS = decltype(stag);
    return dispatch_type(dst_dtype, "eg_scale_copy", [&](auto dtag) {
      using TO = decltype(dtag);
      return dispatch_type(mul_dtype, "eg_scale_copy", [&](auto mtag) {
        using TM = decltype(mtag);
        constexpr int V = 16 / sizeof(TS);
        const TS* sp = static_cast<const TS*>(src);
        TO* dp = static_cast<TO*>(dst);
        const TM* mp = static_cast<const TM*>(mul);
        constexpr int64_t per = 256 * kScaleUnroll;
        if (n % V == 0 && aligned16(src) && ((uintptr_t)dst % (V * sizeof(TO))) == 0) {
          const int64_t np = n / V;
          EG_LAUNCH((scale_copy_kernel<TS, TO, TM, V>), dim3((unsigned)((np + per - 1) / per)),
                    dim3(256), 0, st, sp, dp, np, mp, div);
        } else {
          EG_LAUNCH((scale_copy_kernel<TS, TO, TM, 1>), dim3((unsigned)((n + per - 1) / per)),
                    dim3(256), 0, st, sp, dp, n, mp, div);
        }
        return check_launch("eg_scale_copy");
      });
    });
  });
}
