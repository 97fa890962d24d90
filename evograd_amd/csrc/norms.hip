// RMSNorm, fused residual-add RMSNorm and LayerNorm forward/backward for gfx950.
//
// fused_add_rms_norm follows fused_add_rms_norm_forward_ref
// (src/evograd/ops/level2/fused_add_rms_norm/forward_ref.py:6-16): s = x + r,
// rstd = rsqrt(mean(s^2) + eps), out = s * rstd * weight; its backward
// (declared at fused_add_rms_norm/__init__.py:103-106) is RMSNorm's with s in
// place of x, and dx = dr. Only x, r (the inputs) and rstd are saved: the
// backward forms s again from x and r, which moves the same number of bytes as
// reading a saved s while storing no new row-sized tensor.
//
// RMSNorm follows rmsnorm_forward_ref (src/evograd/ops/level1/rmsnorm/forward_ref.py:6-21)
// and the backward rule at src/evograd/ops/level1/rmsnorm/__init__.py:85-86.
// LayerNorm follows layernorm_forward_ref (src/evograd/ops/level1/layernorm/forward_ref.py:6-23)
// and its autograd backward (grads declared at layernorm/__init__.py:124-171).
//
// Layout: x, y, dy, dx are [rows, hidden] row-major in HBM; weight/bias [hidden];
// the saved statistics (rstd, and mean for LayerNorm) are fp32 [rows].
//
// Ring kernels (every backward, and the forwards for widths the one-wave and
// one-workgroup-per-row kernels do not take): a fixed grid of G workgroups
// walks the rows with stride G. A thread owns the same columns on every row
// (16-byte packs), so weight, bias and the dweight/dbias sums stay in its
// registers. Each workgroup keeps DEPTH rows of loads in flight: a ring slot is
// refilled with the row DEPTH*G further on as soon as its data is in registers,
// before the current row's reduction. Row statistics are reduced with wave
// butterflies and one barrier per sum, through two alternating LDS slots (a
// slot is rewritten only after the next barrier, so no second barrier is needed).
//
// The backward writes one fp32 partial row per workgroup ([G, hidden] per
// parameter); the column-sum kernel adds the G partials of each column in a
// fixed order. No atomics: results are bit-identical from run to run, and G is a
// constant (not the device's CU count), so the summation order is the same on
// every device.
//
// Norm forwards for hidden = 64 x VEC x {1, 2, 4}: one wave per row, the
// statistics reduced by wave butterflies only, so no barrier sits between a row's
// loads and its stores. Rows of 512 packs (4096 bf16 columns) take one 256-thread
// workgroup per row.
#include "eg_common.hpp"

#include <initializer_list>
#include <mutex>

namespace eg {
namespace {

// Workgroups of the backward ring per 512 threads of workgroup width: two
// 512-thread workgroups per CU of an MI355X (256 CUs), each with half the
// forward's ring depth. Measured at [16384, 4096] bf16 (ring + column sum):
// RMSNorm 76.7 us at (256 workgroups, depth 4) -> 74.8 us; LayerNorm 84.6 us at
// (384, 2) -> 79.8 us; 640 and more workgroups are slower. The residual-add
// backward streams three inputs and keeps one workgroup per CU at the full
// depth (its ring at 512 workgroups: 87.1 -> 91.7 us).
constexpr int64_t kRmsBwdBlocks = 512;
constexpr int64_t kLnBwdBlocks = 512;
constexpr int64_t kAddBwdBlocks = 256;
constexpr int64_t kFwdBlocks = 512;

constexpr int64_t bwd_per512(bool ln, bool add) {
  return add ? kAddBwdBlocks : ln ? kLnBwdBlocks : kRmsBwdBlocks;
}

inline int64_t ring_blocks(int64_t rows, int64_t per512, int block) {
  const int64_t g = per512 * (block < 512 ? 512 / block : 1);
  return rows < g ? (rows > 0 ? rows : 1) : g;
}

// Backward rings whose row stream is one 512-thread range (rows of 257-512 packs,
// e.g. 4096 bf16 columns) run two streams per 1024-thread workgroup: the same
// threads in flight as per512 workgroups of 512, half the partial rows. At
// [16384, 4096] bf16 (backward call: ring + column sum, interleaved runs):
// LayerNorm 78.6 -> 74.4 us, RMSNorm 74.3 -> 72.2 us, both with the ring's loads
// issued unconditionally (with the loads under branches the split LayerNorm ring
// was slower, 72.5 -> 85 us). The residual-add ring keeps its own configuration.
inline bool bwd_split(int64_t npack, bool add) { return !add && npack > 256 && npack <= 512; }
inline int64_t split_blocks(int64_t rows, int64_t per512) {
  return ring_blocks((rows + 1) / 2, per512 / 2, 512);
}

// Workgroup width for a row of npack packs: (BLOCK, ITEMS) with BLOCK * ITEMS >= npack.
template <typename F>
bool pick_ring(int64_t npack, F&& f) {
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

inline int ring_block_for(int64_t npack) {
  if (npack <= 64) return 64;
  if (npack <= 128) return 128;
  if (npack <= 256) return 256;
  if (npack <= 512) return 512;
  if (npack <= 1024) return 512;
  return 1024;
}

// Rows in flight per workgroup: deeper for narrow rows, one for very wide ones.
template <int ITEMS> constexpr int ring_depth() { return ITEMS == 1 ? 4 : ITEMS == 2 ? 2 : 1; }

// ------------------------------------------------------------- pack access
template <typename T, int VEC>
__device__ __forceinline__ Pack<T, VEC> ld_raw(const T* __restrict__ p) {
  if constexpr (sizeof(T) * VEC == 16) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    Pack<T, VEC> pk;
    __builtin_memcpy(&pk, &raw, 16);
    return pk;
  } else {
    return *reinterpret_cast<const Pack<T, VEC>*>(p);
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void unpack(const Pack<T, VEC>& pk, float (&f)[VEC]) {
#pragma unroll
  for (int i = 0; i < VEC; ++i) f[i] = to_f32(pk.v[i]);
}

template <typename T, int VEC>
__device__ __forceinline__ void st_vec(T* __restrict__ p, const float (&f)[VEC]) {
  store_vec<T, VEC, true>(p, f);
}

// Sums of N values over each of the SPLIT equal thread ranges of the workgroup
// (one row stream each), with one barrier per call: per-wave butterflies, then
// the wave totals of the range added in wave order from one of two alternating
// LDS slots. Every thread ends with its range's totals.
template <int BLOCK, int N, int SPLIT = 1>
struct SlotSum {
  static constexpr int NW = BLOCK / kWave, NWS = NW / SPLIT;
  float (*slot)[N][NW];  // [2][N][NW] in LDS
  int par;
  __device__ __forceinline__ void operator()(float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = wave_reduce(v[i], SumOp());
    if constexpr (NW > 1) {
      const int lane = threadIdx.x & (kWave - 1);
      const int wid = threadIdx.x / kWave;
      const int w0 = wid / NWS * NWS;  // first wave of this thread's range
      if (lane == 0)
#pragma unroll
        for (int i = 0; i < N; ++i) slot[par][i][wid] = v[i];
      __syncthreads();
#pragma unroll
      for (int i = 0; i < N; ++i) {
        float t = slot[par][i][w0];
#pragma unroll
        for (int q = 1; q < NWS; ++q) t += slot[par][i][w0 + q];
        v[i] = t;
      }
      par ^= 1;
    }
  }
};

// --------------------------------------------------------------- forward
// ADD: the normalised row is s = x + r (fused residual add), formed in fp32.
// SPLIT: row streams per workgroup, as in norm_bwd_ring. Every load is issued
// unconditionally (rows past the end read the last row, dead packs read pack 0).
template <typename T, int VEC, int ITEMS, int BLOCK, int DEPTH, bool LN, bool ADD = false,
          int SPLIT = 1>
__global__ __launch_bounds__(BLOCK) void norm_fwd_ring(const T* __restrict__ x,
                                                       const T* __restrict__ r,
                                                       const T* __restrict__ w,
                                                       const T* __restrict__ b,
                                                       T* __restrict__ y,
                                                       float* __restrict__ mean_out,
                                                       float* __restrict__ rstd_out,
                                                       int64_t rows, int hidden, float eps) {
  static_assert(!(LN && ADD), "the residual add is fused into RMSNorm only");
  static_assert(SPLIT == 1 || SPLIT == 2, "one or two row streams");
  constexpr int SB = BLOCK / SPLIT;
  __shared__ float slots[2][1][BLOCK / kWave];
  SlotSum<BLOCK, 1, SPLIT> bsum{slots, 0};
  const int sid = SPLIT > 1 ? (int)threadIdx.x / SB : 0;
  const int tid = (int)threadIdx.x - sid * SB;
  const int64_t GS = (int64_t)gridDim.x * SPLIT;
  const int64_t first = (int64_t)blockIdx.x * SPLIT;
  const float inv_h = 1.0f / (float)hidden;
  int col[ITEMS], lcol[ITEMS];
  bool live[ITEMS];
  float wv[ITEMS][VEC], bv[ITEMS][VEC];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    col[it] = (it * SB + tid) * VEC;
    live[it] = col[it] < hidden;
    lcol[it] = live[it] ? col[it] : 0;
#pragma unroll
    for (int i = 0; i < VEC; ++i) { wv[it][i] = 0.f; bv[it][i] = 0.f; }
    if (live[it]) {
      unpack<T, VEC>(*reinterpret_cast<const Pack<T, VEC>*>(w + col[it]), wv[it]);
      if (LN) unpack<T, VEC>(*reinterpret_cast<const Pack<T, VEC>*>(b + col[it]), bv[it]);
    }
  }
  const int64_t last = rows - 1;
  Pack<T, VEC> xb[DEPTH][ITEMS], rb[ADD ? DEPTH : 1][ITEMS];
  auto fill = [&](int k, int64_t row) {
    const int64_t rc = row < rows ? row : last;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      xb[k][it] = ld_raw<T, VEC>(x + rc * hidden + lcol[it]);
      if (ADD) rb[ADD ? k : 0][it] = ld_raw<T, VEC>(r + rc * hidden + lcol[it]);
    }
  };
#pragma unroll
  for (int k = 0; k < DEPTH; ++k) fill(k, first + sid + k * GS);
  for (int64_t base = first; base < rows; base += DEPTH * GS) {
#pragma unroll
    for (int k = 0; k < DEPTH; ++k) {
      if (base + k * GS >= rows) break;  // stream 0's row decides for the workgroup
      const int64_t row = base + k * GS + sid;
      const bool here = row < rows;
      float xv[ITEMS][VEC];
#pragma unroll
      for (int it = 0; it < ITEMS; ++it) {
        unpack<T, VEC>(xb[k][it], xv[it]);
        if (ADD) {
          float rv[VEC];
          unpack<T, VEC>(rb[ADD ? k : 0][it], rv);
#pragma unroll
          for (int i = 0; i < VEC; ++i) xv[it][i] += rv[i];
        }
        // dead packs (read from pack 0) are zero
#pragma unroll
        for (int i = 0; i < VEC; ++i) xv[it][i] = live[it] ? xv[it][i] : 0.f;
      }
      fill(k, row + DEPTH * GS);
      float mean = 0.f;
      if (LN) {
        float s[1] = {0.f};
#pragma unroll
        for (int it = 0; it < ITEMS; ++it)
#pragma unroll
          for (int i = 0; i < VEC; ++i) s[0] += xv[it][i];
        bsum(s);
        mean = s[0] * inv_h;
      }
      float q[1] = {0.f};
#pragma unroll
      for (int it = 0; it < ITEMS; ++it)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          // Padding columns hold x = 0 and must not add (0 - mean)^2.
          const float d = live[it] && (col[it] + i < hidden) ? xv[it][i] - mean : 0.f;
          q[0] += d * d;
        }
      bsum(q);
      if (!here) continue;
      const float rstd = rsqrtf(q[0] * inv_h + eps);
      T* yr = y + row * hidden;
#pragma unroll
      for (int it = 0; it < ITEMS; ++it) {
        if (!live[it]) continue;
        float o[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          o[i] = LN ? ((xv[it][i] - mean) * rstd) * wv[it][i] + bv[it][i]
                    : (xv[it][i] * rstd) * wv[it][i];
        st_vec<T, VEC>(yr + col[it], o);
      }
      if (tid == 0) {
        rstd_out[row] = rstd;
        if (LN) mean_out[row] = mean;
      }
    }
  }
}

// RMSNorm forward, one wave per row, for rows of ITEMS x 64 lanes x VEC elements.
// ADD: the normalised row is s = x + r, formed in fp32.
template <typename T, int VEC, int ITEMS, bool ADD = false>
__global__ __launch_bounds__(256) void rmsnorm_fwd_wave(const T* __restrict__ x,
                                                        const T* __restrict__ r,
                                                        const T* __restrict__ w,
                                                        T* __restrict__ y,
                                                        float* __restrict__ rstd_out, int64_t rows,
                                                        float eps) {
  constexpr int H = ITEMS * kWave * VEC;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * H;
  Pack<T, VEC> xp[ITEMS], rp[ADD ? ITEMS : 1];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    xp[it] = ld_raw<T, VEC>(xr + (it * kWave + lane) * VEC);
    if (ADD) rp[ADD ? it : 0] = ld_raw<T, VEC>(r + row * H + (it * kWave + lane) * VEC);
  }
  float sv[ITEMS][VEC];
  float ss = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float v = to_f32(xp[it].v[i]);
      if (ADD) v += to_f32(rp[ADD ? it : 0].v[i]);
      sv[it][i] = v;
      ss += v * v;
    }
  ss = wave_reduce(ss, SumOp());
  const float rs = rsqrtf(ss / (float)H + eps);
  T* yr = y + row * H;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * kWave + lane) * VEC;
    const Pack<T, VEC> wp = *reinterpret_cast<const Pack<T, VEC>*>(w + c);
    float o[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) o[i] = (sv[it][i] * rs) * to_f32(wp.v[i]);
    st_vec<T, VEC>(yr + c, o);
  }
  if (lane == 0) rstd_out[row] = rs;
}

// RMSNorm forward, RPW rows per workgroup of BLOCK threads, each row IT x BLOCK
// packs (4096 bf16 columns at (512, 1)), every thread holding its packs of each of
// the RPW rows; ADD: the normalised row is s = x + r. All loads are issued first
// (rows past the end read the last row again and are not stored), the RPW rows'
// reductions share one barrier. At bf16 [16384, 4096], interleaved: 47.5 us for one
// row per 256-thread workgroup, 46.4 us for two rows per 512-thread workgroup.
template <typename T, int VEC, int IT, int BLOCK, int RPW, bool ADD = false>
__global__ __launch_bounds__(BLOCK) void rmsnorm_fwd_row(const T* __restrict__ x,
                                                         const T* __restrict__ r,
                                                         const T* __restrict__ w,
                                                         T* __restrict__ y,
                                                         float* __restrict__ rstd_out,
                                                         int64_t rows, float eps) {
  constexpr int NW = BLOCK / kWave;
  constexpr int H = IT * BLOCK * VEC;
  __shared__ float red[RPW][NW];
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const int64_t row0 = (int64_t)blockIdx.x * RPW;
  Pack<T, VEC> xp[RPW][IT], rp[ADD ? RPW : 1][ADD ? IT : 1];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int64_t rc = row0 + rr < rows ? row0 + rr : rows - 1;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int64_t off = rc * H + (it * BLOCK + (int)threadIdx.x) * VEC;
      xp[rr][it] = ld_raw<T, VEC>(x + off);
      if (ADD) rp[ADD ? rr : 0][ADD ? it : 0] = ld_raw<T, VEC>(r + off);
    }
  }
  float sv[RPW][IT][VEC];
  float q[RPW];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    q[rr] = 0.f;
#pragma unroll
    for (int it = 0; it < IT; ++it)
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        float v = to_f32(xp[rr][it].v[i]);
        if (ADD) v += to_f32(rp[ADD ? rr : 0][ADD ? it : 0].v[i]);
        sv[rr][it][i] = v;
        q[rr] += v * v;
      }
  }
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) q[rr] += __shfl_xor(q[rr], off, kWave);
  if (lane == 0) {
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) red[rr][wid] = q[rr];
  }
  __syncthreads();
  float rs[RPW];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    float u = red[rr][0];
#pragma unroll
    for (int k = 1; k < NW; ++k) u += red[rr][k];
    rs[rr] = rsqrtf(u / (float)H + eps);
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
    const Pack<T, VEC> wp = *reinterpret_cast<const Pack<T, VEC>*>(w + c);
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      if (row0 + rr >= rows) continue;
      float o[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) o[i] = (sv[rr][it][i] * rs[rr]) * to_f32(wp.v[i]);
      st_vec<T, VEC>(y + (row0 + rr) * H + c, o);
    }
  }
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr)
    if ((int)threadIdx.x == rr && row0 + rr < rows) rstd_out[row0 + rr] = rs[rr];
}

// LayerNorm forward, one wave per row (rows of ITEMS x 64 lanes x VEC elements):
// the row stays in registers; mean, then the centred sum of squares, each one
// wave butterfly; no barrier.
template <typename T, int VEC, int ITEMS>
__global__ __launch_bounds__(256) void layernorm_fwd_wave(const T* __restrict__ x,
                                                          const T* __restrict__ w,
                                                          const T* __restrict__ b,
                                                          T* __restrict__ y,
                                                          float* __restrict__ mean_out,
                                                          float* __restrict__ rstd_out,
                                                          int64_t rows, float eps) {
  constexpr int H = ITEMS * kWave * VEC;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * H;
  Pack<T, VEC> xp[ITEMS];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) xp[it] = ld_raw<T, VEC>(xr + (it * kWave + lane) * VEC);
  float sv[ITEMS][VEC];
  float s = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      sv[it][i] = to_f32(xp[it].v[i]);
      s += sv[it][i];
    }
  const float mean = wave_reduce(s, SumOp()) * (1.0f / (float)H);
  float q = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      sv[it][i] -= mean;
      q += sv[it][i] * sv[it][i];
    }
  const float rs = rsqrtf(wave_reduce(q, SumOp()) * (1.0f / (float)H) + eps);
  T* yr = y + row * H;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * kWave + lane) * VEC;
    const Pack<T, VEC> wp = *reinterpret_cast<const Pack<T, VEC>*>(w + c);
    const Pack<T, VEC> bp = *reinterpret_cast<const Pack<T, VEC>*>(b + c);
    float o[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) o[i] = (sv[it][i] * rs) * to_f32(wp.v[i]) + to_f32(bp.v[i]);
    st_vec<T, VEC>(yr + c, o);
  }
  if (lane == 0) {
    rstd_out[row] = rs;
    mean_out[row] = mean;
  }
}

// LayerNorm forward, RPW rows per workgroup of BLOCK threads, each row IT x BLOCK
// packs (4096 bf16 columns at (512, 1)): mean, then the centred sum of squares,
// each a wave butterfly plus one LDS exchange, shared by the RPW rows (rows past the
// end read the last row again and are not stored). At bf16 [16384, 4096],
// interleaved: 49.5 us for one row per 256-thread workgroup, 50.2 us for one row per
// wave, 47.6 us for two rows per 512-thread workgroup.
template <typename T, int VEC, int IT, int BLOCK, int RPW>
__global__ __launch_bounds__(BLOCK) void layernorm_fwd_row(const T* __restrict__ x,
                                                           const T* __restrict__ w,
                                                           const T* __restrict__ b,
                                                           T* __restrict__ y,
                                                           float* __restrict__ mean_out,
                                                           float* __restrict__ rstd_out,
                                                           int64_t rows, float eps) {
  constexpr int NW = BLOCK / kWave;
  constexpr int H = IT * BLOCK * VEC;
  __shared__ float red[2][RPW][NW];
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  const int64_t row0 = (int64_t)blockIdx.x * RPW;
  Pack<T, VEC> xp[RPW][IT];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    const int64_t rc = row0 + rr < rows ? row0 + rr : rows - 1;
#pragma unroll
    for (int it = 0; it < IT; ++it)
      xp[rr][it] = ld_raw<T, VEC>(x + rc * H + (it * BLOCK + (int)threadIdx.x) * VEC);
  }
  float sv[RPW][IT][VEC];
  float s[RPW];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    s[rr] = 0.f;
#pragma unroll
    for (int it = 0; it < IT; ++it)
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        sv[rr][it][i] = to_f32(xp[rr][it].v[i]);
        s[rr] += sv[rr][it][i];
      }
  }
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) s[rr] += __shfl_xor(s[rr], off, kWave);
  if (lane == 0) {
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) red[0][rr][wid] = s[rr];
  }
  __syncthreads();
  float mean[RPW], q[RPW];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    float t = red[0][rr][0];
#pragma unroll
    for (int k = 1; k < NW; ++k) t += red[0][rr][k];
    mean[rr] = t * (1.0f / (float)H);
    q[rr] = 0.f;
#pragma unroll
    for (int it = 0; it < IT; ++it)
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        sv[rr][it][i] -= mean[rr];
        q[rr] += sv[rr][it][i] * sv[rr][it][i];
      }
  }
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) q[rr] += __shfl_xor(q[rr], off, kWave);
  if (lane == 0) {
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) red[1][rr][wid] = q[rr];
  }
  __syncthreads();
  float rs[RPW];
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) {
    float u = red[1][rr][0];
#pragma unroll
    for (int k = 1; k < NW; ++k) u += red[1][rr][k];
    rs[rr] = rsqrtf(u * (1.0f / (float)H) + eps);
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
    const Pack<T, VEC> wp = *reinterpret_cast<const Pack<T, VEC>*>(w + c);
    const Pack<T, VEC> bp = *reinterpret_cast<const Pack<T, VEC>*>(b + c);
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      if (row0 + rr >= rows) continue;
      float o[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) o[i] = (sv[rr][it][i] * rs[rr]) * to_f32(wp.v[i]) + to_f32(bp.v[i]);
      st_vec<T, VEC>(y + (row0 + rr) * H + c, o);
    }
  }
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr)
    if ((int)threadIdx.x == rr && row0 + rr < rows) {
      rstd_out[row0 + rr] = rs[rr];
      mean_out[row0 + rr] = mean[rr];
    }
}

// -------------------------------------------------------------- backward
// RMSNorm:   xhat = x * rstd, g = dy * w, dx = (g - xhat * mean(g * xhat)) * rstd
// LayerNorm: xhat = (x - mean) * rstd, dx = rstd * (g - mean(g) - xhat * mean(g * xhat))
// dweight += dy * xhat, dbias += dy (per thread, per owned column).
// ADD: the normalised row was s = x + r; it is formed again here from the inputs.
// SPLIT: row streams per workgroup. With SPLIT = 2 the two halves of the workgroup
// walk interleaved rows (stream s of workgroup b takes rows 2b + s, + 2G, ...) and
// add their column sums in LDS (stream 0's + stream 1's) before the one partial row
// of the workgroup is written: half the partial rows of SPLIT = 1 at the same
// number of threads in flight.
template <typename T, int VEC, int ITEMS, int BLOCK, int DEPTH, bool LN, bool ADD = false,
          int SPLIT = 1>
__global__ __launch_bounds__(BLOCK) void norm_bwd_ring(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ res,
    const T* __restrict__ w,
    const float* __restrict__ mean, const float* __restrict__ rstd, T* __restrict__ dx,
    float* __restrict__ partial_w, float* __restrict__ partial_b, int64_t rows, int hidden) {
  static_assert(!(LN && ADD), "the residual add is fused into RMSNorm only");
  static_assert(SPLIT == 1 || SPLIT == 2, "one or two row streams");
  constexpr int NS = LN ? 2 : 1;
  constexpr int SB = BLOCK / SPLIT;  // threads per row stream
  __shared__ float slots[2][NS][BLOCK / kWave];
  SlotSum<BLOCK, NS, SPLIT> bsum{slots, 0};
  const int sid = SPLIT > 1 ? (int)threadIdx.x / SB : 0;
  const int tid = (int)threadIdx.x - sid * SB;
  const int64_t GS = (int64_t)gridDim.x * SPLIT;  // row streams in the grid
  const int64_t first = (int64_t)blockIdx.x * SPLIT;
  const float inv_h = 1.0f / (float)hidden;
  // Every load is issued unconditionally: rows past the end read the last row and
  // dead column packs read pack 0, and their data is never used. With the loads
  // under branches the compiler's load waits are more conservative at the branch
  // joins (the two-stream LayerNorm ring measured 85 against 69 us).
  int col[ITEMS], lcol[ITEMS];
  bool live[ITEMS];
  float wv[ITEMS][VEC], aw[ITEMS][VEC], ab[ITEMS][VEC];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    col[it] = (it * SB + tid) * VEC;
    live[it] = col[it] < hidden;
    lcol[it] = live[it] ? col[it] : 0;
#pragma unroll
    for (int i = 0; i < VEC; ++i) { wv[it][i] = 0.f; aw[it][i] = 0.f; ab[it][i] = 0.f; }
    if (live[it]) unpack<T, VEC>(*reinterpret_cast<const Pack<T, VEC>*>(w + col[it]), wv[it]);
  }
  const int64_t last = rows - 1;
  Pack<T, VEC> xb[DEPTH][ITEMS], gb[DEPTH][ITEMS], resb[ADD ? DEPTH : 1][ITEMS];
  float rb[DEPTH], mb[DEPTH];
  auto fill = [&](int k, int64_t row) {
    const int64_t rc = row < rows ? row : last;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      xb[k][it] = ld_raw<T, VEC>(x + rc * hidden + lcol[it]);
      gb[k][it] = ld_raw<T, VEC>(dy + rc * hidden + lcol[it]);
      if (ADD) resb[ADD ? k : 0][it] = ld_raw<T, VEC>(res + rc * hidden + lcol[it]);
    }
    rb[k] = rstd[rc];
    mb[k] = LN ? mean[rc] : 0.f;
  };
#pragma unroll
  for (int k = 0; k < DEPTH; ++k) fill(k, first + sid + k * GS);
  for (int64_t base = first; base < rows; base += DEPTH * GS) {
#pragma unroll
    for (int k = 0; k < DEPTH; ++k) {
      // Stream 0's row decides for the whole workgroup (every thread reaches the
      // barrier in bsum); stream 1 past the last row takes part with zero sums.
      if (base + k * GS >= rows) break;
      const int64_t row = base + k * GS + sid;
      const bool here = row < rows;
      const float r = rb[k];
      const float mr = LN ? -mb[k] * r : 0.f;  // xhat = x * r + mr
      float xh[ITEMS][VEC], g[ITEMS][VEC];
      float s[NS];
#pragma unroll
      for (int j = 0; j < NS; ++j) s[j] = 0.f;
#pragma unroll
      for (int it = 0; it < ITEMS; ++it) {
        float xv[VEC], gv[VEC];
        unpack<T, VEC>(xb[k][it], xv);
        unpack<T, VEC>(gb[k][it], gv);
        if (ADD) {
          float av[VEC];
          unpack<T, VEC>(resb[ADD ? k : 0][it], av);
#pragma unroll
          for (int i = 0; i < VEC; ++i) xv[i] += av[i];
        }
        // Dead packs (columns past the row, read from pack 0) and a stream's row past
        // the end (read from the last row) take x = dy = 0, so they add nothing to the
        // sums; their outputs are not stored.
        const bool use = here && live[it];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          xv[i] = use ? xv[i] : 0.f;
          gv[i] = use ? gv[i] : 0.f;
          const float h = LN ? __builtin_fmaf(xv[i], r, mr) : xv[i] * r;
          aw[it][i] = __builtin_fmaf(gv[i], h, aw[it][i]);
          if (LN) ab[it][i] += gv[i];
          const float gg = gv[i] * wv[it][i];
          s[0] = __builtin_fmaf(gg, h, s[0]);
          if (LN) s[1] += gg;
          xh[it][i] = h;
          g[it][i] = gg;
        }
      }
      fill(k, row + DEPTH * GS);
      bsum(s);
      if (!here) continue;
      // dx = r * (g - mean(g) - xhat * mean(g * xhat)) = g * r + (xhat * c2 + c1)
      const float c2 = -(s[0] * inv_h) * r;
      const float c1 = LN ? -(s[1] * inv_h) * r : 0.f;
      T* dxr = dx + row * hidden;
#pragma unroll
      for (int it = 0; it < ITEMS; ++it) {
        if (!live[it]) continue;
        float o[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          o[i] = __builtin_fmaf(g[it][i], r, __builtin_fmaf(xh[it][i], c2, c1));
        st_vec<T, VEC>(dxr + col[it], o);
      }
    }
  }
  if constexpr (SPLIT > 1) {
    // Stream 1 hands its column sums to stream 0 through LDS; stream 0 adds them
    // to its own (that order) and writes the workgroup's partial row.
    __shared__ float comb[NS][SB * ITEMS * VEC];
    if (sid == 1) {
#pragma unroll
      for (int it = 0; it < ITEMS; ++it)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          comb[0][(it * SB + tid) * VEC + i] = aw[it][i];
          if (LN) comb[NS - 1][(it * SB + tid) * VEC + i] = ab[it][i];
        }
    }
    __syncthreads();
    if (sid == 1) return;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it)
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        aw[it][i] += comb[0][(it * SB + tid) * VEC + i];
        if (LN) ab[it][i] += comb[NS - 1][(it * SB + tid) * VEC + i];
      }
  }
  float* pw = partial_w + (int64_t)blockIdx.x * hidden;
  float* pb = LN ? partial_b + (int64_t)blockIdx.x * hidden : nullptr;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    if (!live[it]) continue;
    if (col[it] + VEC <= hidden) {
      store_f32<float, VEC>(pw + col[it], aw[it]);
      if (LN) store_f32<float, VEC>(pb + col[it], ab[it]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i)
        if (col[it] + i < hidden) {
          pw[col[it] + i] = aw[it][i];
          if (LN) pb[col[it] + i] = ab[it][i];
        }
    }
  }
}

// ------------------------------------------------- stage 2: column sums
// out[c] = sum_{g=0..G-1} partial[g][c]. A wave owns 4 adjacent columns; lane l
// adds the partial rows l, l + 64, l + 128, ... in ascending order (batches of 8
// loads issued together), then the 64 lane totals are combined by a butterfly.
// The order is fixed, so the result is bit-identical on every run.
// blockIdx.y selects the parameter (0: p0 -> o0, 1: p1 -> o1).
template <typename T>
__global__ __launch_bounds__(256) void colsum_kernel(const float* __restrict__ p0,
                                                     const float* __restrict__ p1,
                                                     T* __restrict__ o0, T* __restrict__ o1,
                                                     int G, int hidden) {
  constexpr int kBatch = 8;
  const int lane = threadIdx.x & (kWave - 1);
  const int c = ((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6)) * 4;
  if (c >= hidden) return;  // whole wave leaves together
  const float* p = blockIdx.y == 0 ? p0 : p1;
  T* o = blockIdx.y == 0 ? o0 : o1;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if ((hidden & 3) == 0) {
    for (int g0 = lane; g0 < G; g0 += kWave * kBatch) {
      float4 v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int g = g0 + kWave * i;
        v[i] = g < G ? *reinterpret_cast<const float4*>(p + (int64_t)g * hidden + c)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        acc[0] += v[i].x; acc[1] += v[i].y; acc[2] += v[i].z; acc[3] += v[i].w;
      }
    }
  } else {
    for (int g = lane; g < G; g += kWave)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (c + i < hidden) acc[i] += p[(int64_t)g * hidden + c + i];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = wave_reduce(acc[i], SumOp());
  if (lane == 0)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (c + i < hidden) o[c + i] = from_f32<T>(acc[i]);
}

// Column sums of G partial rows when hidden % 4 == 0: a 1024-thread workgroup per
// 4 * CQ columns. Lane (row group rg = lane / CQ, column quad cq = lane % CQ) of
// wave w adds rows w * RG + rg, + 16 RG, + 32 RG, ... (RG = 64 / CQ row groups per
// wave; all of a lane's loads issued together, each wave instruction reading RG
// rows x 16 CQ contiguous bytes); the row groups are combined by lane exchanges
// and the 16 waves through LDS, in a fixed order.
template <typename T, int CQ>
__global__ __launch_bounds__(1024) void colsum_wide_kernel(const float* __restrict__ p0,
                                                           const float* __restrict__ p1,
                                                           T* __restrict__ o0, T* __restrict__ o1,
                                                           int G, int hidden) {
  constexpr int RG = kWave / CQ, kBatch = 8;
  __shared__ float4 red[16][CQ];
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
  const int cq = lane % CQ, rg = lane / CQ;
  const int c = ((int)blockIdx.x * CQ + cq) * 4;
  const float* p = blockIdx.y == 0 ? p0 : p1;
  T* o = blockIdx.y == 0 ? o0 : o1;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (c < hidden) {
    for (int g0 = w * RG + rg; g0 < G; g0 += 16 * RG * kBatch) {
      float4 v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int g = g0 + 16 * RG * i;
        v[i] = g < G ? *reinterpret_cast<const float4*>(p + (int64_t)g * hidden + c)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        acc.x += v[i].x; acc.y += v[i].y; acc.z += v[i].z; acc.w += v[i].w;
      }
    }
  }
#pragma unroll
  for (int off = CQ; off < kWave; off <<= 1) {
    acc.x += __shfl_xor(acc.x, off, kWave);
    acc.y += __shfl_xor(acc.y, off, kWave);
    acc.z += __shfl_xor(acc.z, off, kWave);
    acc.w += __shfl_xor(acc.w, off, kWave);
  }
  if (rg == 0) red[w][cq] = acc;
  __syncthreads();
  if (threadIdx.x < CQ) {
    const int cc = ((int)blockIdx.x * CQ + (int)threadIdx.x) * 4;
    float4 s = red[0][threadIdx.x];
#pragma unroll
    for (int ww = 1; ww < 16; ++ww) {
      const float4 t = red[ww][threadIdx.x];
      s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
    }
    if (cc < hidden) {
      o[cc + 0] = from_f32<T>(s.x);
      o[cc + 1] = from_f32<T>(s.y);
      o[cc + 2] = from_f32<T>(s.z);
      o[cc + 3] = from_f32<T>(s.w);
    }
  }
}

// 32 columns per workgroup (measured at 512 x 4096 partial rows: 7.9 us cold for
// one parameter, 10.3 us for two, against 8.8 and 14.0 us for colsum_kernel).
constexpr int kColsumQuads = 8;

template <typename T>
int launch_colsum(const float* p0, const float* p1, T* o0, T* o1, int nparams, int G,
                  int hidden, hipStream_t st, const char* what) {
  const int quads = (hidden + 3) / 4;
  // The partial rows come from the same workspace base, so 16-byte alignment of
  // p0 and a hidden divisible by 4 make every row's float4 loads aligned.
  if (hidden % 4 == 0 && aligned16(p0) && aligned16(p1)) {
    EG_LAUNCH((colsum_wide_kernel<T, kColsumQuads>),
              dim3((unsigned)((quads + kColsumQuads - 1) / kColsumQuads), (unsigned)nparams),
              dim3(1024), 0, st, p0, p1, o0, o1, G, hidden);
  } else {
    EG_LAUNCH((colsum_kernel<T>), dim3((unsigned)((quads + 3) / 4), (unsigned)nparams),
              dim3(256), 0, st, p0, p1, o0, o1, G, hidden);
  }
  return check_launch(what);
}

// ------------------------------------------------------------- dispatch
template <typename T, int VEC, bool LN, bool ADD = false>
struct FwdRing {
  const T *x, *r, *w, *b; T* y; float *mean, *rstd; int64_t rows; int hidden; float eps;
  hipStream_t st;
  template <int BLOCK, int ITEMS> bool go() {
    const int64_t G = ring_blocks(rows, kFwdBlocks, BLOCK);
    EG_LAUNCH((norm_fwd_ring<T, VEC, ITEMS, BLOCK, ring_depth<ITEMS>(), LN, ADD>),
              dim3((unsigned)G), dim3(BLOCK), 0, st, x, r, w, b, y, mean, rstd, rows, hidden, eps);
    return true;
  }
};

template <typename T, int VEC, bool LN, bool ADD = false>
struct BwdRing {
  const T *dy, *x, *res, *w; const float *mean, *rstd; T* dx; float *pw, *pb; int64_t rows;
  int hidden; hipStream_t st;
  template <int BLOCK, int ITEMS> bool go() {
    // Two workgroups per CU share its registers: half the forward's ring depth.
    constexpr int D = ADD ? ring_depth<ITEMS>()
                          : (ring_depth<ITEMS>() > 1 ? ring_depth<ITEMS>() / 2 : 1);
    if constexpr (BLOCK == 512 && ITEMS == 1 && !ADD) {
      // Two 512-thread row streams per 1024-thread workgroup (see bwd_split).
      const int64_t G = split_blocks(rows, bwd_per512(LN, ADD));
      EG_LAUNCH((norm_bwd_ring<T, VEC, 1, 1024, D, LN, ADD, 2>), dim3((unsigned)G), dim3(1024),
                0, st, dy, x, res, w, mean, rstd, dx, pw, pb, rows, hidden);
      return true;
    }
    const int64_t G = ring_blocks(rows, bwd_per512(LN, ADD), BLOCK);
    EG_LAUNCH((norm_bwd_ring<T, VEC, ITEMS, BLOCK, D, LN, ADD>), dim3((unsigned)G), dim3(BLOCK),
              0, st, dy, x, res, w, mean, rstd, dx, pw, pb, rows, hidden);
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

// Partial rows of the backward for a given dtype width (must match the launch).
int64_t bwd_blocks(int64_t rows, int64_t hidden, bool ln, bool add, bool vec, int elem) {
  const int64_t npack = vec ? (hidden + (16 / elem) - 1) / (16 / elem) : hidden;
  if (bwd_split(npack, add)) return split_blocks(rows, bwd_per512(ln, add));
  return ring_blocks(rows, bwd_per512(ln, add), ring_block_for(npack));
}

}  // namespace
}  // namespace eg

using namespace eg;

// Workspace: nparams x [G, hidden] fp32 partials. G depends on the workgroup
// width, which depends on the dtype; the size returned covers the widest case
// (the 16-bit vector path has the narrowest workgroups, hence the largest G).
static size_t norm_workspace_bytes(int64_t rows, int64_t hidden, bool ln) {
  if (rows <= 0 || hidden <= 0) return 0;
  int64_t G = 0;
  for (int elem : {2, 4})
    for (bool vec : {true, false}) {
      for (bool add : {false, true}) {
        if (ln && add) continue;
        const int64_t g = bwd_blocks(rows, hidden, ln, add, vec, elem);
        if (g > G) G = g;
      }
    }
  return (size_t)(ln ? 2 : 1) * (size_t)G * (size_t)hidden * sizeof(float);
}

extern "C" size_t eg_rmsnorm_workspace_bytes(int64_t rows, int64_t hidden) {
  return norm_workspace_bytes(rows, hidden, false);
}

extern "C" size_t eg_layernorm_workspace_bytes(int64_t rows, int64_t hidden) {
  return norm_workspace_bytes(rows, hidden, true);
}

// RMSNorm of x (ADD = false) or of x + r (ADD = true); r may be null otherwise.
template <bool ADD>
static int rms_fwd_impl(const char* name, const void* x, const void* r, const void* weight,
                        void* y, float* rstd, int64_t rows, int64_t hidden, float eps, int dtype,
                        void* stream) {
  clear_error();
  if (check_norm_dims(name, rows, hidden)) return 1;
  if (rows == 0) return 0;
  if (!x || (ADD && !r) || !weight || !y || !rstd) { set_error("%s: null pointer", name); return 1; }
  hipStream_t st = as_stream(stream);
  return EG_DISPATCH_FLOAT(dtype, name, [&] {
    using T = scalar_t;
    constexpr int V = 16 / sizeof(T);
    const int h = (int)hidden;
    const T* xp = (const T*)x;
    const T* rp = (const T*)r;
    const T* wp = (const T*)weight;
    T* yp = (T*)y;
    bool ok = true;
    const int wave_items = h / (kWave * V);
    const bool vec = vec_ok<T>(h, {x, weight, y}) && (!ADD || aligned16(r));
    if (vec && h % (kWave * V) == 0 &&
        (wave_items == 1 || wave_items == 2 || wave_items == 4 || wave_items == 8)) {
      const unsigned grid = (unsigned)((rows + 3) / 4);
      switch (wave_items) {
        case 1: EG_LAUNCH((rmsnorm_fwd_wave<T, V, 1, ADD>), dim3(grid), dim3(256), 0, st, xp, rp, wp, yp, rstd, rows, eps); break;
        case 2: EG_LAUNCH((rmsnorm_fwd_wave<T, V, 2, ADD>), dim3(grid), dim3(256), 0, st, xp, rp, wp, yp, rstd, rows, eps); break;
        case 4: EG_LAUNCH((rmsnorm_fwd_wave<T, V, 4, ADD>), dim3(grid), dim3(256), 0, st, xp, rp, wp, yp, rstd, rows, eps); break;
        // rows of 512 packs: two rows per 512-thread workgroup (ADD: one row per 256
        // threads, the configuration its residual loads were measured at)
        default:
          if (ADD)
            EG_LAUNCH((rmsnorm_fwd_row<T, V, 2, 256, 1, ADD>), dim3((unsigned)rows), dim3(256), 0, st, xp, rp, wp, yp, rstd, rows, eps);
          else
            EG_LAUNCH((rmsnorm_fwd_row<T, V, 1, 512, 2, ADD>), dim3((unsigned)((rows + 1) / 2)), dim3(512), 0, st, xp, rp, wp, yp, rstd, rows, eps);
          break;
      }
    } else if (vec) {
      FwdRing<T, V, false, ADD> f{xp, rp, wp, nullptr, yp, nullptr, rstd, rows, h, eps, st};
      ok = pick_ring((h + V - 1) / V, f);
    } else {
      FwdRing<T, 1, false, ADD> f{xp, rp, wp, nullptr, yp, nullptr, rstd, rows, h, eps, st};
      ok = pick_ring(h, f);
    }
    if (!ok) { set_error("%s: hidden=%d too wide", name, h); return 1; }
    return check_launch(name);
  });
}

template <bool ADD>
static int rms_bwd_impl(const char* name, const void* dy, const void* x, const void* r,
                        const void* weight, const float* rstd, void* dx, void* dweight,
                        void* workspace, int64_t rows, int64_t hidden, int dtype, void* stream) {
  clear_error();
  if (check_norm_dims(name, rows, hidden)) return 1;
  if (!dweight) { set_error("%s: null dweight", name); return 1; }
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    // Empty batch: dweight is a sum over no rows.
    size_t es = dtype == EG_F32 ? 4 : 2;
    return zero_fill(dweight, (size_t)hidden * es, st, name);
  }
  if (!dy || !x || (ADD && !r) || !weight || !rstd || !dx || !workspace) {
    set_error("%s: null pointer", name);
    return 1;
  }
  return EG_DISPATCH_FLOAT(dtype, name, [&] {
    using T = scalar_t;
    constexpr int V = 16 / sizeof(T);
    const int h = (int)hidden;
    float* part = (float*)workspace;
    const bool vec = vec_ok<T>(h, {dy, x, weight, dx}) && (!ADD || aligned16(r));
    bool ok;
    if (vec) {
      BwdRing<T, V, false, ADD> f{(const T*)dy, (const T*)x, (const T*)r, (const T*)weight, nullptr,
                                  rstd, (T*)dx, part, nullptr, rows, h, st};
      ok = pick_ring((h + V - 1) / V, f);
    } else {
      BwdRing<T, 1, false, ADD> f{(const T*)dy, (const T*)x, (const T*)r, (const T*)weight, nullptr,
                                  rstd, (T*)dx, part, nullptr, rows, h, st};
      ok = pick_ring(h, f);
    }
    if (!ok) { set_error("%s: hidden=%d too wide", name, h); return 1; }
    if (int rc = check_launch(name)) return rc;
    const int G = (int)bwd_blocks(rows, h, false, ADD, vec, (int)sizeof(T));
    return launch_colsum<T>(part, part, (T*)dweight, (T*)dweight, 1, G, h, st, name);
  });
}

extern "C" int eg_rmsnorm_fwd(const void* x, const void* weight, void* y, float* rstd,
                              int64_t rows, int64_t hidden, float eps, int dtype,
                              void* stream) {
  return rms_fwd_impl<false>("eg_rmsnorm_fwd", x, nullptr, weight, y, rstd, rows, hidden, eps,
                             dtype, stream);
}

extern "C" int eg_rmsnorm_bwd(const void* dy, const void* x, const void* weight,
                              const float* rstd, void* dx, void* dweight, void* workspace,
                              int64_t rows, int64_t hidden, int dtype, void* stream) {
  return rms_bwd_impl<false>("eg_rmsnorm_bwd", dy, x, nullptr, weight, rstd, dx, dweight,
                             workspace, rows, hidden, dtype, stream);
}

extern "C" int eg_fused_add_rmsnorm_fwd(const void* x, const void* r, const void* weight,
                                        void* y, float* rstd, int64_t rows, int64_t hidden,
                                        float eps, int dtype, void* stream) {
  return rms_fwd_impl<true>("eg_fused_add_rmsnorm_fwd", x, r, weight, y, rstd, rows, hidden, eps,
                            dtype, stream);
}

extern "C" int eg_fused_add_rmsnorm_bwd(const void* dout, const void* x, const void* r,
                                        const void* weight, const float* rstd, void* ds,
                                        void* dweight, void* workspace, int64_t rows,
                                        int64_t hidden, int dtype, void* stream) {
  return rms_bwd_impl<true>("eg_fused_add_rmsnorm_bwd", dout, x, r, weight, rstd, ds, dweight,
                            workspace, rows, hidden, dtype, stream);
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
    bool ok = true;
    const int wave_items = h / (kWave * V);
    const bool vec = vec_ok<T>(h, {x, weight, bias, y});
    if (vec && h % (kWave * V) == 0 &&
        (wave_items == 1 || wave_items == 2 || wave_items == 4 || wave_items == 8)) {
      const unsigned grid = (unsigned)((rows + 3) / 4);
      const T* xp = (const T*)x;
      const T* wp = (const T*)weight;
      const T* bp = (const T*)bias;
      T* yp = (T*)y;
      switch (wave_items) {
        case 1: EG_LAUNCH((layernorm_fwd_wave<T, V, 1>), dim3(grid), dim3(256), 0, st, xp, wp, bp, yp, mean, rstd, rows, eps); break;
        case 2: EG_LAUNCH((layernorm_fwd_wave<T, V, 2>), dim3(grid), dim3(256), 0, st, xp, wp, bp, yp, mean, rstd, rows, eps); break;
        case 4: EG_LAUNCH((layernorm_fwd_wave<T, V, 4>), dim3(grid), dim3(256), 0, st, xp, wp, bp, yp, mean, rstd, rows, eps); break;
        // rows of 512 packs: two rows per 512-thread workgroup
        default: EG_LAUNCH((layernorm_fwd_row<T, V, 1, 512, 2>), dim3((unsigned)((rows + 1) / 2)), dim3(512), 0, st, xp, wp, bp, yp, mean, rstd, rows, eps); break;
      }
    } else if (vec) {
      FwdRing<T, V, true> f{(const T*)x, nullptr, (const T*)weight, (const T*)bias, (T*)y, mean, rstd, rows, h, eps, st};
      ok = pick_ring((h + V - 1) / V, f);
    } else {
      FwdRing<T, 1, true> f{(const T*)x, nullptr, (const T*)weight, (const T*)bias, (T*)y, mean, rstd, rows, h, eps, st};
      ok = pick_ring(h, f);
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
    const bool vec = vec_ok<T>(h, {dy, x, weight, dx});
    const int G = (int)bwd_blocks(rows, h, true, false, vec, (int)sizeof(T));
    float* pw = (float*)workspace;
    float* pb = pw + (int64_t)G * h;
    bool ok;
    if (vec) {
      BwdRing<T, V, true> f{(const T*)dy, (const T*)x, nullptr, (const T*)weight, mean, rstd, (T*)dx, pw, pb, rows, h, st};
      ok = pick_ring((h + V - 1) / V, f);
    } else {
      BwdRing<T, 1, true> f{(const T*)dy, (const T*)x, nullptr, (const T*)weight, mean, rstd, (T*)dx, pw, pb, rows, h, st};
      ok = pick_ring(h, f);
    }
    if (!ok) { set_error("eg_layernorm_bwd: hidden=%d too wide", h); return 1; }
    if (int rc = check_launch("eg_layernorm_bwd")) return rc;
    return launch_colsum<T>(pw, pb, (T*)dweight, (T*)dbias, 2, G, h, st,
                            "eg_layernorm_bwd(colsum)");
  });
}

// ------------------------------------------- small-shape backward, one launch
// For few rows (the reference's small regime, under 4096 tokens) the ring backward
// and its column sum are two latency-bound launches: at bf16 [1024, 4096] 10.2 and
// 4.0 us, for 25 MB. This kernel does the whole backward in one launch with no
// partial rows, in two kinds of workgroups:
//   column workgroups (first): 4 packs of columns each, 64 row lanes; lane walks
//     rows rl, rl + 64, ... (8 rows' loads in flight) summing dy * xhat (and dy) per
//     column in fp32 (compensated), then the 64 lane sums are added in a fixed
//     pairwise tree ->
//     dweight (dbias): bitwise repeatable, and read from dy, x and the saved row
//     statistics alone;
//   row workgroups: one row each, two passes over the row (the second from L2):
//     the row sums, then dx.
// dy and x are read twice (once per role), which at these sizes the 256 MB
// Infinity Cache serves; for wide batches the ring, which reads them once, is
// the program to use.
constexpr int kSmallBlock = 256, kSmallPacks = 4, kSmallLanes = kSmallBlock / kSmallPacks;
constexpr int kSmallUnroll = 8;  // rows of a lane whose loads are issued together

template <typename T, int VEC, bool LN>
__global__ __launch_bounds__(kSmallBlock) void norm_bwd_small(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ w,
    const float* __restrict__ mean, const float* __restrict__ rstd, T* __restrict__ dx,
    T* __restrict__ dweight, T* __restrict__ dbias, int64_t rows, int hidden, int ncolwg) {
  __shared__ float part[2][kSmallLanes][kSmallPacks * VEC];
  __shared__ float red[2][kSmallBlock / kWave];
  const int t = threadIdx.x;
  if ((int)blockIdx.x < ncolwg) {
    const int p = t % kSmallPacks, rl = t / kSmallPacks;
    const int c0 = ((int)blockIdx.x * kSmallPacks + p) * VEC;
    const bool live = c0 < hidden;
    // Compensated (Kahan) sums per lane, then a pairwise tree over the 64 lanes: a
    // lane's rows are summed in order with their rounding errors carried, so the
    // result stays within a few units of the exact column sum even where the rows
    // cancel (the ring's many short partial rows give the same by splitting).
    float sw[VEC], sb[VEC], cw[VEC], cb[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) { sw[i] = 0.f; sb[i] = 0.f; cw[i] = 0.f; cb[i] = 0.f; }
    auto kahan = [](float& s, float& c, float v) {
      const float y = v - c;
      const float t2 = s + y;
      c = (t2 - s) - y;
      s = t2;
    };
    if (live) {
      // kSmallUnroll rows per batch, all their loads issued before the sums (rows
      // past the end load row 0 and are skipped)
      for (int64_t r0 = rl; r0 < rows; r0 += (int64_t)kSmallLanes * kSmallUnroll) {
        float g[kSmallUnroll][VEC], xv[kSmallUnroll][VEC], rs[kSmallUnroll], mu[kSmallUnroll];
#pragma unroll
        for (int u = 0; u < kSmallUnroll; ++u) {
          const int64_t r = r0 + (int64_t)u * kSmallLanes;
          const int64_t rc = r < rows ? r : 0;
          load_f32<T, VEC>(dy + rc * hidden + c0, g[u]);
          load_f32<T, VEC>(x + rc * hidden + c0, xv[u]);
          rs[u] = rstd[rc];
          mu[u] = LN ? mean[rc] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kSmallUnroll; ++u) {
          if (r0 + (int64_t)u * kSmallLanes >= rows) break;
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            kahan(sw[i], cw[i], g[u][i] * ((xv[u][i] - mu[u]) * rs[u]));
            if (LN) kahan(sb[i], cb[i], g[u][i]);
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      part[0][rl][p * VEC + i] = sw[i] - cw[i];
      if (LN) part[1][rl][p * VEC + i] = sb[i] - cb[i];
    }
    __syncthreads();
    if (t < kSmallPacks * VEC) {
      const int col = (int)blockIdx.x * kSmallPacks * VEC + t;
      float a[kSmallLanes], b[kSmallLanes];
#pragma unroll
      for (int l = 0; l < kSmallLanes; ++l) {
        a[l] = part[0][l][t];
        b[l] = LN ? part[1][l][t] : 0.f;
      }
#pragma unroll
      for (int w2 = kSmallLanes / 2; w2 >= 1; w2 >>= 1)
#pragma unroll
        for (int l = 0; l < w2; ++l) {
          a[l] += a[l + w2];
          if (LN) b[l] += b[l + w2];
        }
      if (col < hidden) {
        dweight[col] = from_f32<T>(a[0]);
        if (LN) dbias[col] = from_f32<T>(b[0]);
      }
    }
    return;
  }
  const int64_t r = (int64_t)blockIdx.x - ncolwg;
  const T* dyr = dy + r * hidden;
  const T* xr = x + r * hidden;
  const float rs = rstd[r], mu = LN ? mean[r] : 0.f;
  // pass 1: sum(g) (LayerNorm) and sum(g * xhat), g = dy * w
  float sa = 0.f, sg = 0.f;
  for (int c = t * VEC; c < hidden; c += kSmallBlock * VEC) {
    float g[VEC], xv[VEC], wv[VEC];
    load_f32<T, VEC>(dyr + c, g);
    load_f32<T, VEC>(xr + c, xv);
    load_f32<T, VEC>(w + c, wv);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float gi = g[i] * wv[i];
      sa = __builtin_fmaf(gi, (xv[i] - mu) * rs, sa);
      if (LN) sg += gi;
    }
  }
  sa = wave_reduce(sa, SumOp());
  if (LN) sg = wave_reduce(sg, SumOp());
  if ((t & (kWave - 1)) == 0) {
    red[0][t / kWave] = sa;
    red[1][t / kWave] = sg;
  }
  __syncthreads();
  float ta = red[0][0], tg = red[1][0];
#pragma unroll
  for (int k = 1; k < kSmallBlock / kWave; ++k) {
    ta += red[0][k];
    tg += red[1][k];
  }
  const float inv_h = 1.0f / (float)hidden;
  const float mgx = ta * inv_h, mg = LN ? tg * inv_h : 0.f;
  // pass 2: dx = rstd * (g - mean(g) - xhat * mean(g * xhat))   (RMSNorm: no mean(g))
  for (int c = t * VEC; c < hidden; c += kSmallBlock * VEC) {
    float g[VEC], xv[VEC], wv[VEC], o[VEC];
    load_f32<T, VEC>(dyr + c, g);
    load_f32<T, VEC>(xr + c, xv);
    load_f32<T, VEC>(w + c, wv);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float xh = (xv[i] - mu) * rs;
      o[i] = (g[i] * wv[i] - mg - xh * mgx) * rs;
    }
    store_f32<T, VEC>(dx + r * hidden + c, o);
  }
}

template <bool LN>
static int norm_bwd_small_impl(const char* name, const void* dy, const void* x,
                               const void* weight, const float* mean, const float* rstd,
                               void* dx, void* dweight, void* dbias, int64_t rows,
                               int64_t hidden, int dtype, void* stream) {
  clear_error();
  if (check_norm_dims(name, rows, hidden)) return 1;
  if (!dweight || (LN && !dbias)) { set_error("%s: null dweight/dbias", name); return 1; }
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    const size_t es = dtype == EG_F32 ? 4 : 2;
    if (int rc = zero_fill(dweight, (size_t)hidden * es, st, name)) return rc;
    return LN ? zero_fill(dbias, (size_t)hidden * es, st, name) : 0;
  }
  if (!dy || !x || !weight || (LN && !mean) || !rstd || !dx) {
    set_error("%s: null pointer", name);
    return 1;
  }
  if (rows > 0x7fffffff - 65536) {
    set_error("%s: rows=%lld exceeds the launch grid", name, (long long)rows);
    return 1;
  }
  return EG_DISPATCH_FLOAT(dtype, name, [&] {
    using T = scalar_t;
    constexpr int V = 16 / sizeof(T);
    const int h = (int)hidden;
    auto go = [&](auto vc) {
      constexpr int VC = decltype(vc)::value;
      const int ncol = (h + kSmallPacks * VC - 1) / (kSmallPacks * VC);
      EG_LAUNCH((norm_bwd_small<T, VC, LN>), dim3((unsigned)(ncol + rows)), dim3(kSmallBlock), 0,
                st, (const T*)dy, (const T*)x, (const T*)weight, mean, rstd, (T*)dx, (T*)dweight,
                (T*)dbias, rows, h, ncol);
      return check_launch(name);
    };
    if (vec_ok<T>(h, {dy, x, weight, dx})) return go(std::integral_constant<int, V>{});
    return go(std::integral_constant<int, 1>{});
  });
}

extern "C" int eg_rmsnorm_bwd_small(const void* dy, const void* x, const void* weight,
                                    const float* rstd, void* dx, void* dweight, int64_t rows,
                                    int64_t hidden, int dtype, void* stream) {
  return norm_bwd_small_impl<false>("eg_rmsnorm_bwd_small", dy, x, weight, nullptr, rstd, dx,
                                    dweight, nullptr, rows, hidden, dtype, stream);
}

extern "C" int eg_layernorm_bwd_small(const void* dy, const void* x, const void* weight,
                                      const float* mean, const float* rstd, void* dx,
                                      void* dweight, void* dbias, int64_t rows, int64_t hidden,
                                      int dtype, void* stream) {
  return norm_bwd_small_impl<true>("eg_layernorm_bwd_small", dy, x, weight, mean, rstd, dx,
                                   dweight, dbias, rows, hidden, dtype, stream);
}

// ------------------------------------------------- allocation-free backward
// eg_rmsnorm_bwd_noalloc runs eg_rmsnorm_bwd's kernels with the partial rows in
// `scratch`, a device-resident array of the library (one copy per GPU, held
// until the process ends), for callers that cannot allocate. Every workgroup of
// the ring writes its whole partial row before the column sum reads it, so the
// array needs no clearing between calls. Calls that overlap on one GPU share the
// array and race.
static __device__ __align__(256) unsigned char scratch[EG_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};  // device address of `scratch`, per device

// The device address of `scratch` on the current device. The array's name is a
// host-side stand-in; its device address comes from hipGetSymbolAddress, called
// once per device with that device current.
int scratch_address(const char* name, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("%s: no usable current device (%d)", name, dev);
    return 1;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", name, dev,
                hipGetErrorString(e));
      return 1;
    }
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return 0;
}
}  // namespace

extern "C" int eg_rmsnorm_bwd_noalloc(const void* dy, const void* x, const void* weight,
                                      const float* rstd, void* dx, void* dweight, int64_t rows,
                                      int64_t hidden, int dtype, void* stream) {
  static const char* name = "eg_rmsnorm_bwd_noalloc";
  // rms_bwd_impl clears the error slot (and starts the kernel-timing hook's call)
  if (check_norm_dims(name, rows, hidden)) return 1;
  const size_t need = norm_workspace_bytes(rows, hidden, false);
  if (need > (size_t)EG_NOALLOC_SCRATCH_BYTES) {
    set_error("%s: rows=%lld hidden=%lld need %zu bytes of partial rows, more than the "
              "%d-byte scratch; use eg_rmsnorm_bwd with a workspace", name, (long long)rows,
              (long long)hidden, need, EG_NOALLOC_SCRATCH_BYTES);
    return 1;
  }
  const hipStream_t st = as_stream(stream);
  if (st) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || hipGetStreamDeviceId(st) != cur) {
      set_error("%s: the stream belongs to device %d, not the current device %d", name,
                hipGetStreamDeviceId(st), cur);
      return 1;
    }
  }
  void* part = nullptr;
  if (rows > 0 && scratch_address(name, &part)) return 1;
  return rms_bwd_impl<false>(name, dy, x, nullptr, weight, rstd, dx, dweight, part, rows, hidden,
                             dtype, stream);
}
