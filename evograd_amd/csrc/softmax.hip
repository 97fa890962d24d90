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
// 16-bit rows up to 131072 columns are held on chip split between LDS and registers
// (softmax_fwd_lds / softmax_bwd_lds), so both passes read HBM once. Wider rows take a
// two-read path: the row's logsumexp
// (forward) or sum(dy * y) (backward) in one read, then y = exp(x - lse) or
// dx = y * (dy - sum) in a second read and the write.
#include "rowwise.hpp"

namespace eg {
namespace {

// Buffer resource over one row: packs past its end read as zero and their stores are
// dropped, so 16-byte rows are loaded and stored with no branch per pack (measured
// on fp32 [4096, 4096]: forward and backward 1% faster than branch-guarded loads).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
constexpr int kNtAux = 2;  // buffer access cache policy: non-temporal

template <typename T, int VEC, int ITEMS, int BLOCK, bool NT>
__device__ __forceinline__ void load_row(const T* __restrict__ row, int cols, float fill,
                                         float (&v)[ITEMS][VEC]) {
  if constexpr (NT) {  // 16-byte packs
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(row, cols * (int)sizeof(T));
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
      typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 raw = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, c * (int)sizeof(T), 0, kNtAux));
      Pack<T, VEC> pk;
      __builtin_memcpy(&pk, &raw, 16);
#pragma unroll
      for (int i = 0; i < VEC; ++i) v[it][i] = c + i < cols ? to_f32(pk.v[i]) : fill;
    }
  } else {
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
}

template <typename T, int VEC, int ITEMS, int BLOCK, bool NT>
__device__ __forceinline__ void store_row(T* __restrict__ row, int cols,
                                          const float (&v)[ITEMS][VEC]) {
  if constexpr (NT) {
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(row, cols * (int)sizeof(T));
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
      Pack<T, VEC> pk;
#pragma unroll
      for (int i = 0; i < VEC; ++i) pk.v[i] = from_f32<T>(v[it][i]);
      typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
      u32x4 raw;
      __builtin_memcpy(&raw, &pk, 16);
      __builtin_amdgcn_raw_buffer_store_b128(raw, rs, c * (int)sizeof(T), 0, kNtAux);
    }
  } else {
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int c = (it * BLOCK + (int)threadIdx.x) * VEC;
      if (c < cols) store_vec<T, VEC, NT>(row + c, v[it]);
    }
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
  // exp(x - m) as exp2 of one FMA (x log2e - m log2e): measured 3% faster than expf
  // on fp32 [4096, 4096] at 512 threads per row
  constexpr float kL2e = 1.4426950408889634f;
  const float ml = m * kL2e;
  float s = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      v[it][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(v[it][i], kL2e, -ml));
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

// ---- 16-bit rows of up to 131072 columns (the Llama-3 vocabulary): every input
// byte is read from HBM once. A row is held on chip as raw 16-byte packs, split
// between LDS (packs 0..LITEMS-1 of every thread, filled by buffer->LDS loads) and
// registers, and converted to fp32 again in each pass; the empty asm statements keep
// the compiler from hoisting fp32 copies of the register packs across the
// reductions. All loads go through buffer resources bounded by the row's bytes, so
// none sits under a branch: packs past the row read as zeros, in registers and in
// LDS alike (the bounded-access rules in eg_common.hpp), and are masked in the
// reductions.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

template <typename T>
__device__ __forceinline__ void unpack8(const u32x4& raw, float (&f)[8]) {
  Pack<T, 8> pk;
  __builtin_memcpy(&pk, &raw, 16);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = to_f32(pk.v[i]);
}

template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const T* row, int cols) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(row), (short)0, cols * (int)sizeof(T),
                                           0x00020000);
}
constexpr int kNtLoad = 2;  // buffer-load cache policy: non-temporal

// Forward: 512-thread workgroups, two per CU (72 KB of LDS and at most 128 VGPRs each),
// so that one workgroup's stores overlap the other's loads (one 1024-thread
// workgroup per CU holding the row in registers: 405.6 us against 393.8 us at
// [4096, 128256] bf16). The LDS packs are read one ahead of their use, each read's
// address tied to the previous pack, so that the reads are not all hoisted into
// registers at once.
template <typename T, int ITEMS, int LITEMS, int BLOCK>
__global__ __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(4, 4)))
void softmax_fwd_lds(const T* __restrict__ x, T* __restrict__ y, int cols) {
  static_assert(sizeof(T) == 2, "16-bit rows");
  constexpr int RI = ITEMS - LITEMS;
  __shared__ float red[2][BLOCK / kWave];
  __shared__ __align__(16) uint16_t xs[LITEMS * BLOCK * 8];
  const int64_t off = (int64_t)blockIdx.x * cols;
  const int tid = threadIdx.x, w = tid >> 6;
  const __amdgpu_buffer_rsrc_t rx = row_rsrc(x + off, cols);
#pragma unroll
  for (int it = 0; it < LITEMS; ++it)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void*)(xs + (it * BLOCK + w * kWave) * 8),
                                             16, (it * BLOCK + tid) * 16, 0, 0, kNtLoad);
  u32x4 xr[RI];
#pragma unroll
  for (int it = 0; it < RI; ++it)
    xr[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           rx, ((it + LITEMS) * BLOCK + tid) * 16, 0, kNtLoad));
  // A lane reads only the LDS slots its own loads wrote: no barrier needed.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  auto pass = [&](auto&& fn) {
#pragma unroll
    for (int it = LITEMS; it < ITEMS; ++it) fn(it, xr[it - LITEMS]);
    const char* base = reinterpret_cast<const char*>(xs);
    u32x4 cur = *reinterpret_cast<const u32x4*>(base + tid * 16);
#pragma unroll
    for (int it = 0; it < LITEMS; ++it) {
      u32x4 nxt = cur;
      if (it + 1 < LITEMS) {
        int an = ((it + 1) * BLOCK + tid) * 16;
        asm volatile("" : "+v"(an) : "v"(cur));
        nxt = *reinterpret_cast<const u32x4*>(base + an);
      }
      fn(it, cur);
      cur = nxt;
    }
  };
  // The row's max and sum of exponentials in one pass (online): a running max m
  // (log2 domain) and the sum of exp2(v - m) over this thread's packs, rescaled when
  // a pack raises m; then the (m, sum) pairs over the workgroup. Against a max pass
  // followed by a sum pass (one pass, one reduction and one read of the LDS packs
  // fewer): 395.0 -> 383.5 us at [4096, 128256] bf16, outputs within one bf16 unit
  // (13.5k of 525M differ by one: the fp32 sum's rounding order). Packs past the row
  // are skipped (cols % 8 == 0 here, so a pack is wholly in or out); a pack with no
  // finite value while m is still -inf adds nothing.
  constexpr float L2E = rowwise::kLog2e;
  float m = -INFINITY, s = 0.f;
  pass([&](int it, const u32x4& p) {
    if ((it * BLOCK + tid) * 8 >= cols) return;
    float f[8];
    unpack8<T>(p, f);
    float pm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      f[i] *= L2E;
      pm = fmaxf(pm, f[i]);
    }
    if (pm > m) {
      s *= __builtin_amdgcn_exp2f(m - pm);
      m = pm;
    }
    if (m == -INFINITY) return;
#pragma unroll
    for (int i = 0; i < 8; ++i) s += __builtin_amdgcn_exp2f(f[i] - m);
  });
  // (m, s) combined over the lanes (butterfly) and then the waves in order
  auto comb = [](float& m1, float& s1, float m2, float s2) {
    const float mm = fmaxf(m1, m2);
    if (mm == -INFINITY) return;
    s1 = s1 * __builtin_amdgcn_exp2f(m1 - mm) + s2 * __builtin_amdgcn_exp2f(m2 - mm);
    m1 = mm;
  };
#pragma unroll
  for (int o = kWave / 2; o >= 1; o >>= 1) {
    const float m2 = __shfl_xor(m, o, kWave), s2 = __shfl_xor(s, o, kWave);
    comb(m, s, m2, s2);
  }
  if ((tid & (kWave - 1)) == 0) {
    red[0][w] = m;
    red[1][w] = s;
  }
  __syncthreads();
  float mt = red[0][0], st = red[1][0];
#pragma unroll
  for (int k = 1; k < BLOCK / kWave; ++k) comb(mt, st, red[0][k], red[1][k]);
#pragma unroll
  for (int it = 0; it < RI; ++it) asm volatile("" : "+v"(xr[it]));
  // log2 of the row's normaliser, max included (a row of -inf: -inf + log2(0), NaN
  // outputs as torch gives)
  const float ll = mt + log2f(st);
  pass([&](int it, const u32x4& p) {
    const int c = (it * BLOCK + tid) * 8;
    if (c < cols) {
      float f[8];
      unpack8<T>(p, f);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        f[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(f[i], rowwise::kLog2e, -ll));
      store_vec<T, 8, true>(y + off + c, f);
    }
  });
}
constexpr int kFwdRowItems = 32, kFwdRowLds = 9, kFwdRowBlock = 512;

// Backward: one 1024-thread workgroup per CU. y in registers (64 VGPRs); dy's first
// LITEMS packs per thread in LDS (144 KB), the rest in registers: y and dy are both
// read once (against y in registers and dy read twice: 651.3 -> 544.2 us at
// [4096, 128256] bf16, 1.21x -> 1.0x of the algorithmic bytes).
template <typename T, int ITEMS, int LITEMS, int BLOCK>
__global__ __launch_bounds__(BLOCK) void softmax_bwd_lds(const T* __restrict__ y,
                                                         const T* __restrict__ dy,
                                                         T* __restrict__ dx, int cols) {
  static_assert(sizeof(T) == 2, "16-bit rows");
  constexpr int RI = ITEMS - LITEMS;
  __shared__ float lds[BLOCK / kWave];
  __shared__ __align__(16) uint16_t dys[LITEMS * BLOCK * 8];
  const int64_t off = (int64_t)blockIdx.x * cols;
  const int tid = threadIdx.x, w = tid >> 6;
  const __amdgpu_buffer_rsrc_t ry = row_rsrc(y + off, cols);
  const __amdgpu_buffer_rsrc_t rg = row_rsrc(dy + off, cols);
#pragma unroll
  for (int it = 0; it < LITEMS; ++it)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (lds_void*)(dys + (it * BLOCK + w * kWave) * 8),
                                             16, (it * BLOCK + tid) * 16, 0, 0, kNtLoad);
  u32x4 yr[ITEMS], gr[RI];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it)
    yr[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           ry, (it * BLOCK + tid) * 16, 0, kNtLoad));
#pragma unroll
  for (int it = 0; it < RI; ++it)
    gr[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           rg, ((it + LITEMS) * BLOCK + tid) * 16, 0, kNtLoad));
  // LDS slots past the row hold zeros written by the bounded buffer->LDS loads, and
  // the register loads return zeros there too (eg_common.hpp), so they add nothing
  // to sum(dy * y).
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // own LDS slots only: no barrier
  auto gpack = [&](int it) -> u32x4 {
    return it < LITEMS ? *reinterpret_cast<const u32x4*>(dys + (it * BLOCK + tid) * 8)
                       : gr[it - LITEMS];
  };
  float d = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    float f[8], g[8];
    unpack8<T>(yr[it], f);
    unpack8<T>(gpack(it), g);
#pragma unroll
    for (int i = 0; i < 8; ++i) d += f[i] * g[i];
  }
  d = block_reduce<BLOCK>(d, SumOp(), lds);
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) asm volatile("" : "+v"(yr[it]));
#pragma unroll
  for (int it = 0; it < RI; ++it) asm volatile("" : "+v"(gr[it]));
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int c = (it * BLOCK + tid) * 8;
    if (c < cols) {
      float f[8], g[8];
      unpack8<T>(yr[it], f);
      unpack8<T>(gpack(it), g);
#pragma unroll
      for (int i = 0; i < 8; ++i) g[i] = f[i] * (g[i] - d);
      store_vec<T, 8, true>(dx + off + c, g);
    }
  }
}
constexpr int kBwdRowItems = 16, kBwdRowLds = 9, kBwdRowBlock = 1024;

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
  // rows of 513-1024 packs: 512 threads of 2 packs (fp32 [*, 4096]: 25.7 against
  // 26.2 us for 256 threads of 4)
  if (npack > 512 && npack <= 1024) {
    l.template go<512, 2>();
    return;
  }
  if (pick_row_config(npack, l)) return;
  if constexpr (sizeof(T) == 2 && VEC == 8) {
    if (npack <= (int64_t)kFwdRowItems * kFwdRowBlock) {
      EG_LAUNCH((softmax_fwd_lds<T, kFwdRowItems, kFwdRowLds, kFwdRowBlock>), dim3((unsigned)rows),
                dim3(kFwdRowBlock), 0, st, x, y, cols);
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
  // rows of 513-1024 packs: 512 threads of 2 packs, as in the forward (fp32
  // [4096, 4096], interleaved: 33.4 against 34.1 us for 256 threads of 4)
  if (npack > 512 && npack <= 1024) {
    l.template go<512, 2>();
    return;
  }
  if (pick_row_config(npack, l)) return;
  if constexpr (sizeof(T) == 2 && VEC == 8) {
    if (npack <= (int64_t)kBwdRowItems * kBwdRowBlock) {
      EG_LAUNCH((softmax_bwd_lds<T, kBwdRowItems, kBwdRowLds, kBwdRowBlock>), dim3((unsigned)rows),
                dim3(kBwdRowBlock), 0, st, y, dy, dx, cols);
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
