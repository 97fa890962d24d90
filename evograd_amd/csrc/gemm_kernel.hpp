// Dense products of the fused linear cross entropy on gfx950 MFMA.
//
// fused_linear_cross_entropy (src/evograd/ops/level2/fused_linear_cross_entropy/
// forward_ref.py:23-35, gradients declared at fused_linear_cross_entropy/
// __init__.py:91-152) needs three rows x hidden x vocab products:
//   logits = x W^T     A = x [M][K],        B = W [N][K]      (both K-contiguous)
//   dx     = dl W      A = dl [M][K],       B = W [K][N]      (B N-contiguous)
//   dW     = dl^T x    A = dl^T: dl [K][M], B = x [K][N]      (both K-major)
// One kernel template covers them: C[M][N] = sum_k A[m][k] B[k][n], fp32
// accumulation, with each operand either K-contiguous (rows of the operand's
// matrix run along k) or K-major (rows run along m or n).
//
// Block tile 256 x 256 x 64 for 4 waves (2 x 2, each wave 128 x 128: sixteen
// 32 x 32 accumulator tiles, 256 fp32 registers per lane, held in AGPRs at one
// wave per SIMD). Per 64-deep k step a workgroup stages a 256 x 64 slice of each
// operand in LDS (32 KB each, double-buffered: 128 KB), filled by direct
// buffer->LDS loads (16 bytes per lane, no VGPR staging) issued about one step
// ahead. A step's one barrier sits before its last substep: the wave waits for its
// own loads of the next slice and for its reads of the current one, then issues,
// among the last 16 MFMAs, the A loads of the slice after next into the buffer
// just released and the reads for the next step's first substep; the next
// slice's B loads follow every second MFMA of an earlier substep. A load
// instruction holds the wave's issue for several cycles: issued as one block
// before the MFMAs they left the matrix unit idle (measured at the benchmark
// sizes, logits 44.6 -> 49.0%, dx 44.8 -> 52.8%, dweight 42.2 -> 48.7% of bf16
// peak), and the barrier before the last substep takes the LDS read latency out
// of the step boundary (a further 1-5%).
// Operands reach the MFMA v_mfma_f32_32x32x16_{bf16,f16} (lane l: row/column
// l%32, k = 8(l/32) .. +7) as
//   K-contiguous slice [256][64]: one ds_read_b128 per operand, 16-byte chunks
//     XOR-swizzled by (row >> 1) & 7 so the 16 rows a read serves at a time fall
//     in 16 distinct bank groups;
//   K-major slice [64][256]: two ds_read_b64_tr_b16 per operand (lane gets 4
//     consecutive k of one column each), chunks XOR-swizzled by 4 (k & 3) so the
//     4 rows of one transposed read fall in 4 distinct 64-byte quarters.
// Per k step a wave issues 64 MFMAs against 32 (K-contiguous) or 64 (K-major)
// LDS reads. The MFMA takes the B operand as its first (row) operand, so each
// accumulator holds a tile of C^T: lane l keeps row l%32 of C and four
// consecutive columns per register group, stored as one 16-byte (fp32) or 8-byte
// (16-bit) vector.
//
// Bounds: rows of an operand past its end are outside the buffer resource's range
// and read as zero, so M, N and a K-major operand's K may be ragged. A K-contiguous
// operand must have K % 64 == 0 (its rows are padded by the caller) and every row
// stride must be a multiple of 8 elements, with 16-byte aligned bases (checked by
// the host). Workgroups walk the output tiles m-fastest within contiguous ranges
// per XCD, so the workgroups in flight on one XCD share B panels in its L2.
//
// The kernels live in this header; gemm.hip holds the host side and the
// gemm_inst_*.hip sources instantiate the kernels.
#pragma once

#include "eg_common.hpp"

#include <algorithm>
#include <type_traits>

namespace eg {
namespace gk {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
#define EG_LDS __attribute__((address_space(3)))

template <typename T> struct GM;
template <> struct GM<bf16_t> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct GM<f16_t> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int kBM = 256, kBN = 256, kBK = 64, kThreads = 256;
constexpr int kSliceElems = 256 * 64;  // one operand slice: 32 KB of 16-bit values

__device__ __forceinline__ int gwave() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}
__device__ __forceinline__ int swz_kc(int row) { return (row >> 1) & 7; }   // 8 chunks/row
__device__ __forceinline__ int swz_km(int krow) { return (krow & 3) << 2; }  // 32 chunks/row

// Buffer resource over [base, base + bytes); reads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const uint16_t* base, int64_t bytes) {
  const int64_t cap = 0x7fffffff;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base), (short)0,
                                           (int)(bytes < cap ? (bytes > 0 ? bytes : 0) : cap),
                                           0x00020000);
}

// Loads one 256 x 64 operand slice into LDS. K-contiguous (KC): the slice is rows
// r0 .. r0+255 of a [rows][ld] matrix, columns k0 .. k0+63. K-major: rows
// k0 .. k0+63 of a [K][ld] matrix, columns c0 .. c0+255.
template <bool KC>
struct SliceLoader {
  int voff[8];
  __device__ __forceinline__ void init(int64_t ld) {
    const int w = gwave(), lane = threadIdx.x & 63;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int p = (it * 4 + w) * 64 + lane;  // LDS chunk (16 bytes) this lane fills
      if (KC) {
        const int r = p >> 3, c = (p & 7) ^ swz_kc(r);
        voff[it] = (int)(((int64_t)r * ld + c * 8) * 2);
      } else {
        const int k = p >> 5, c = (p & 31) ^ swz_km(k);
        voff[it] = (int)(((int64_t)k * ld + c * 8) * 2);
      }
    }
  }
  // `base` = first element of the slice; `bytes` = bytes from there to the end of
  // the matrix.
  __device__ __forceinline__ void load(const uint16_t* base, int64_t bytes,
                                       uint16_t* lds) const {
    const __amdgpu_buffer_rsrc_t rs = rsrc(base, bytes);
    const int w = gwave();
#pragma unroll
    for (int it = 0; it < 8; ++it)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (EG_LDS void*)(lds + (it * 4 + w) * 512), 16,
                                               voff[it], 0, 0, 0);
  }
};

// Operands of the 32 x 32 x 16 MFMA from a slice: for block i (32 rows, or
// columns, starting at w0 + 32 i) and substep s (k = 16 s .. +15), lane l takes row
// w0 + 32 i + l%32, k 8(l/32) .. +7. The per-lane element offsets are computed once,
// so each read is a register plus an immediate:
//   K-contiguous: the swizzle depends on the lane and s only (32 i leaves
//     (row >> 1) & 7 unchanged): off[s], block i adds 32 rows = 2048 elements;
//   K-major: ds_read_b64_tr_b16 (within each 16-lane group, lane j addresses row
//     base + j/4, columns 4(j%4) .. +3 of a 16-column group and receives column j of
//     rows base .. base+3); two reads (rows +0..3, +4..7) give k in natural order.
//     The swizzle depends on the lane only (k & 3 is the same for every s and for
//     the +4 read): off[i], substep s adds 16 rows = 4096 elements.
template <bool KC>
struct OperandReader {
  int off[4];
  __device__ __forceinline__ void init(int w0, int lane) {
    const int l32 = lane & 31, hh = lane >> 5;
    if constexpr (KC) {
      const int row = w0 + l32;
#pragma unroll
      for (int s = 0; s < 4; ++s) off[s] = row * 64 + (((2 * s + hh) ^ swz_kc(row)) << 3);
    } else {
      const int m = lane & 15, gs = (lane >> 4) & 1;
      const int k0 = 8 * hh + (m >> 2);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = w0 + 32 * i + 16 * gs + 4 * (m & 3);
        off[i] = k0 * 256 + (((col >> 3) ^ swz_km(k0)) << 3) + (col & 7);
      }
    }
  }
  template <typename V>
  __device__ __forceinline__ V read(const uint16_t* lds, int i, int s) const {
    if constexpr (KC) {
      return *reinterpret_cast<const V*>(lds + off[s] + i * 2048);
    } else {
      const uint16_t* p = lds + off[i] + s * 4096;
      const i16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((EG_LDS i16x4*)p);
      const i16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((EG_LDS i16x4*)(p + 1024));
      V r;
      __builtin_memcpy(&r, &a, 8);
      __builtin_memcpy(reinterpret_cast<char*>(&r) + 8, &b, 8);
      return r;
    }
  }
};

template <typename TC> __device__ __forceinline__ void put(TC* p, float v);
template <> __device__ __forceinline__ void put<float>(float* p, float v) { *p = v; }
template <> __device__ __forceinline__ void put<bf16_t>(bf16_t* p, float v) { *p = from_f32<bf16_t>(v); }
template <> __device__ __forceinline__ void put<f16_t>(f16_t* p, float v) { *p = from_f32<f16_t>(v); }

// Output tile of workgroup i: XCD i % 8 takes a contiguous range of the tile
// order. The order walks groups of kGroupM m-tiles: within a group, m fastest,
// then n. The 32 workgroups in flight on one XCD then cover about 4 x 8 tiles
// and share 4 A and 8 B slices per k step in that XCD's L2 (measured against
// m-fastest over all m tiles, 16 x 2 in flight: logits 4.38 -> 3.96 ms at
// 4096 x 128256 x 4096).
constexpr int kGroupM = 4;
__device__ __forceinline__ void tile_decode(int t, int tiles_m, int tiles, int& tm, int& tn) {
  const int tiles_n = tiles / tiles_m;
  const int g = t / (kGroupM * tiles_n);
  const int gm = min(kGroupM, tiles_m - g * kGroupM);
  const int r = t - g * kGroupM * tiles_n;
  tm = g * kGroupM + r % gm;
  tn = r / gm;
}
// Workgroups [0, round8(head)) take tiles [0, head) whole, XCD-contiguously as
// above. A split tail (tail > 0): workgroup head + j takes tile head + j % tail and
// k part j / tail. Returns the tile order index t (-1: no tile) and the part.
__device__ __forceinline__ int tile_index(int head, int tail, int& kpart) {
  const int i = blockIdx.x;
  kpart = -1;
  if (tail > 0 && i >= head) {
    const int j = i - head;
    kpart = j / tail;
    return head + j % tail;
  }
  const int per = (head + 7) / 8;
  const int t = (i % 8) * per + i / 8;
  return t < head ? t : -1;
}
constexpr int kTileElems = kBM * kBN;  // one fp32 partial tile of a split tail

// Softmax epilogue of the logits product (SMX): target [M], per-group statistics
// [M][nh2][2] and the target logits [M].
struct SmxArgs {
  const int64_t* target;
  float* hstats;
  float* tlogit;
  int nh2;
};

// Operand segments: the product's operands may be concatenations, along one of
// M, N or K, of up to kMaxSegs separate buffers that share a row stride (the
// projections of one input by several weights, or their gradients, as one product).
// Segment s covers [start[s], start[s + 1]) of that dimension; every start is a
// multiple of the tile (256 along M or N, 64 along K), so a workgroup's tile (M, N)
// or a k slice (K) lies in one segment. a/b/c[s] point at element (start[s]) of
// the segmented dimension of each operand that the dimension indexes (null: that
// operand is the single buffer passed as usual): along M, A (rows m of a k-contiguous
// A, columns of a k-major one) and C (rows); along N, B and C (columns); along K,
// A and B.
constexpr int kMaxSegs = 4;
enum SegDim { kSegNone = 0, kSegM = 1, kSegN = 2, kSegK = 3 };
struct SegArgs {
  int dim, n;
  int start[kMaxSegs + 1];
  const void* a[kMaxSegs];
  const void* b[kMaxSegs];
  void* c[kMaxSegs];
};
__device__ __forceinline__ int seg_of(const SegArgs& g, int idx) {
  int s = 0;
#pragma unroll
  for (int i = 1; i < kMaxSegs; ++i) s += (i < g.n && idx >= g.start[i]) ? 1 : 0;
  return s;
}
// Base, shift and element bound of one operand [rows][ld]: element (r, c) of the
// product's view is at base + r * ld + c - shift, and bytes past `end` elements
// (from base) read as zero.
struct OpView {
  const uint16_t* base;
  int64_t shift, end;
};
template <bool KC>
__device__ __forceinline__ OpView seg_view(const uint16_t* plain, int64_t rows, int64_t ld,
                                           const SegArgs& g, const void* const* tab, bool along_k,
                                           int idx) {
  OpView v{plain, 0, rows * ld};
  if (g.dim == kSegNone || (g.dim == kSegK) != along_k) return v;
  const int s = seg_of(g, idx);
  if (!tab[s]) return v;
  const int64_t st = g.start[s], en = g.start[s + 1];
  v.base = (const uint16_t*)tab[s];
  // the segmented dimension runs along the operand's rows (k-contiguous operand
  // segmented along M or N; k-major along K) or along its columns
  const bool rows_seg = KC != along_k;
  v.shift = rows_seg ? st * ld : st;
  v.end = rows_seg ? (en - st) * ld : rows * ld;
  return v;
}

// Address of C element (row, col) under the segments of C (see SegArgs).
template <typename TC>
__device__ __forceinline__ TC* c_at(TC* C, int64_t ldc, const SegArgs& g, int row, int col) {
  if (g.dim == kSegM || g.dim == kSegN) {
    const int sg = seg_of(g, g.dim == kSegM ? row : col);
    if (g.c[sg])
      return (TC*)g.c[sg] + ((int64_t)row * ldc + col -
                             (g.dim == kSegM ? (int64_t)g.start[sg] * ldc : g.start[sg]));
  }
  return C + (int64_t)row * ldc + col;
}

// One accumulator value read out of its AGPR. The "a" operand keeps the
// accumulators in AGPRs through the k loop when an epilogue feeds them to VALU
// work (otherwise the allocator moves them to VGPRs and spills inside the loop).
__device__ __forceinline__ float acc_read(float x) {
  float r;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(r) : "a"(x));
  return r;
}

// Substep of a k step that carries the B loads of the next slice (the A loads
// follow the step's barrier, in substep 3): measured at the benchmark sizes,
// substep 1 suits the product with both operands K-major, substep 0 the others.
template <bool AKC, bool BKC> struct LoadSpread { static constexpr int b_substep = !AKC && !BKC ? 1 : 0; };

template <typename T, bool AKC, bool BKC, typename TC, bool SMX = false, int SEG = 0>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                 TC* C, int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc,
                 int64_t a_rows, int64_t b_rows, int tiles_m, int tiles, int vec_c,
                 SmxArgs smx, const void* R, int64_t ldr, int r_f32, int kt_per,
                 float* __restrict__ part, int head, int tail, SegArgs seg) {
  using v8 = typename GM<T>::v8;
  // Two separate buffers per operand, selected at compile time in the unrolled k
  // loop: the LDS reads of one buffer provably do not alias the loads in flight
  // into the other, so they need not wait for them.
  __shared__ __align__(16) uint16_t As0[kSliceElems], As1[kSliceElems];
  __shared__ __align__(16) uint16_t Bs0[kSliceElems], Bs1[kSliceElems];
  int kpart;
  const int t_idx = tile_index(head, tail, kpart);
  if (t_idx < 0) return;
  int tm, tn;
  tile_decode(t_idx, tiles_m, tiles, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const int lane = threadIdx.x & 63, w = gwave();
  const int wm = (w >> 1) * 128, wn = (w & 1) * 128;

  SliceLoader<AKC> la;
  SliceLoader<BKC> lb;
  la.init(lda);
  lb.init(ldb);
  // Split K: with part != nullptr and no split tail, workgroup row blockIdx.y takes
  // k slices [kb, kb + kt_per) and writes its fp32 partial tile to the [M][N] slab
  // part[blockIdx.y]; a split tail's workgroup (kpart >= 0) takes slices of part
  // kpart and writes a tile-major partial (splitk_tail_reduce_kernel sums them).
  const bool partial = part && (tail == 0 || kpart >= 0);
  const int nk_all = (K + kBK - 1) / kBK;
  const int kb = partial ? (tail ? kpart : (int)blockIdx.y) * kt_per : 0;
  const int nk = partial ? min(nk_all, kb + kt_per) : nk_all;
  // The k loop runs an even number of steps (two per iteration, one per buffer). A
  // slice at or past nk loads through an empty buffer range, which fills its LDS
  // slots with zeros (the bounded-access rules in eg_common.hpp): the step past the
  // range, when its length is odd, adds zeros.
  const int nk2 = kb + (nk - kb) + ((nk - kb) & 1);

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  // Operand registers ping-pong over the substeps of every step: substep s of a
  // step computes from set s & 1 while set (s + 1) & 1 is read, and the reads for
  // the next step's substep 0 are issued during substep 3, after the step's
  // barrier, so no step starts by waiting for LDS reads.
  OperandReader<AKC> ra;
  OperandReader<BKC> rb;
  ra.init(wm, lane);
  rb.init(wn, lane);
  // LDS read instructions per substep (a K-major operand takes two per block).
  constexpr int NR = 4 * (AKC ? 1 : 2) + 4 * (BKC ? 1 : 2);
  // substep that carries the B loads of the next slice
  constexpr int QB = LoadSpread<AKC, BKC>::b_substep;
  v8 a[2][4], b[2][4];
  auto rd = [&](int set, const uint16_t* as, const uint16_t* bs, int s) {
#pragma unroll
    for (int i = 0; i < 4; ++i) a[set][i] = ra.template read<v8>(as, i, s);
#pragma unroll
    for (int j = 0; j < 4; ++j) b[set][j] = rb.template read<v8>(bs, j, s);
  };
  auto mma16 = [&](int set) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = GM<T>::mma(b[set][j], a[set][i], acc[i][j]);
  };
  // A barrier without a memory fence: the waits before it are explicit, and the
  // fence of __syncthreads() would also wait for the slice loads in flight.
  auto bar = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // Plain operands: the slice's buffer range runs to the end of the matrix.
  const int64_t a_end = a_rows * lda, b_end = b_rows * ldb;
  auto loadA_plain = [&](int kt, uint16_t* as) {
    const int k0 = kt * kBK;
    const int64_t oa = AKC ? (int64_t)m0 * lda + k0 : (int64_t)k0 * lda + m0;
    la.load(A + oa, kt < nk ? (a_end - oa) * 2 : 0, as);
  };
  auto loadB_plain = [&](int kt, uint16_t* bs) {
    const int k0 = kt * kBK;
    const int64_t ob = BKC ? (int64_t)n0 * ldb + k0 : (int64_t)k0 * ldb + n0;
    lb.load(B + ob, kt < nk ? (b_end - ob) * 2 : 0, bs);
  };
  // Segmented operands (SEG = 1: along M or N, the tile's segment is fixed for the
  // workgroup; SEG = 2: along K, each operand keeps a running view that advances when
  // a slice crosses into the next segment: slices are loaded in increasing k, and the
  // argument table is read only on a crossing, so the loop holds no indexed argument
  // read, whose scalar-memory wait would also wait for the LDS reads in flight).
  OpView va = seg_view<AKC>(A, a_rows, lda, seg, seg.a, false, m0);
  OpView vb = seg_view<BKC>(B, b_rows, ldb, seg, seg.b, false, n0);
  int sa = 0, sb = 0, next_a = 0x7fffffff, next_b = 0x7fffffff;
  if constexpr (SEG == 2) {
    auto first = [&](auto kcc, const void* t0, int64_t rows, int64_t ld, OpView& v, int& nx) {
      constexpr bool KC = decltype(kcc)::value;
      if (!t0) return;  // this operand is the plain buffer
      v.base = (const uint16_t*)t0;
      v.shift = 0;
      v.end = KC ? rows * ld : (int64_t)seg.start[1] * ld;
      nx = seg.n > 1 ? seg.start[1] : 0x7fffffff;
    };
    first(std::integral_constant<bool, AKC>{}, seg.a[0], a_rows, lda, va, next_a);
    first(std::integral_constant<bool, BKC>{}, seg.b[0], b_rows, ldb, vb, next_b);
  }
  auto advance = [&](auto kcc, const void* const* tab, int64_t rows, int64_t ld, int k0,
                     OpView& v, int& si, int& nx) {
    constexpr bool KC = decltype(kcc)::value;
    while (k0 >= nx) {  // uniform and rare: at most kMaxSegs - 1 times per operand
      ++si;
      const int64_t st = seg.start[si], en = seg.start[si + 1];
      v.base = (const uint16_t*)tab[si];
      v.shift = KC ? st : st * ld;
      v.end = KC ? rows * ld : (en - st) * ld;
      nx = si + 1 < seg.n ? seg.start[si + 1] : 0x7fffffff;
    }
  };
  auto loadA_seg = [&](int kt, uint16_t* as) {
    const int k0 = kt * kBK;
    if constexpr (SEG == 2)
      advance(std::integral_constant<bool, AKC>{}, seg.a, a_rows, lda, k0, va, sa, next_a);
    const int64_t oa = (AKC ? (int64_t)m0 * lda + k0 : (int64_t)k0 * lda + m0) - va.shift;
    la.load(va.base + oa, kt < nk ? (va.end - oa) * 2 : 0, as);
  };
  auto loadB_seg = [&](int kt, uint16_t* bs) {
    const int k0 = kt * kBK;
    if constexpr (SEG == 2)
      advance(std::integral_constant<bool, BKC>{}, seg.b, b_rows, ldb, k0, vb, sb, next_b);
    const int64_t ob = (BKC ? (int64_t)n0 * ldb + k0 : (int64_t)k0 * ldb + n0) - vb.shift;
    lb.load(vb.base + ob, kt < nk ? (vb.end - ob) * 2 : 0, bs);
  };
  // The segmented form is a separate instantiation (SEG): its per-slice selection
  // costs the plain products 7-19% when compiled into the same kernel.
  auto loadA = [&](int kt, uint16_t* as) {
    if constexpr (SEG != 0) loadA_seg(kt, as);
    else loadA_plain(kt, as);
  };
  auto loadB = [&](int kt, uint16_t* bs) {
    if constexpr (SEG != 0) loadB_seg(kt, bs);
    else loadB_plain(kt, bs);
  };
  loadA(kb, As0);
  loadB(kb, Bs0);
  loadA(kb + 1, As1);
  __builtin_amdgcn_s_waitcnt(0xF78);  // vmcnt(8): slice kb has landed
  bar();
  rd(0, As0, Bs0, 0);
  // Step kt on buffer (as, bs): substeps 0-2 with the B loads of slice kt + 1 (into
  // the other buffer) spread over the MFMAs of substep QB; the wait for this wave's
  // loads of slice kt + 1 and for the reads of substep 3; the barrier (slice kt + 1
  // complete, every wave done reading this buffer); substep 3 with the A loads of
  // slice kt + 2 into this buffer and the reads of the next step's substep 0. Each
  // load slot follows every second MFMA.
  auto step = [&](auto bufc, int kt) {
    constexpr bool odd = decltype(bufc)::value;
    uint16_t* as = odd ? As1 : As0;
    uint16_t* bs = odd ? Bs1 : Bs0;
    uint16_t* an = odd ? As0 : As1;
    uint16_t* bn = odd ? Bs0 : Bs1;
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (QB == 0) loadB(kt + 1, bn);
    rd(1, as, bs, 1);
    mma16(0);
    if constexpr (QB == 1) loadB(kt + 1, bn);
    rd(0, as, bs, 2);
    mma16(1);
    rd(1, as, bs, 3);
    mma16(0);
#pragma unroll
    for (int s = 0; s < 3; ++s)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (s == QB && (q & 1)) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
        // NR <= 16: at most one read after each MFMA
        if (((q + 1) * NR) / 16 != (q * NR) / 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
    bar();
    loadA(kt + 2, as);
    rd(0, an, bn, 0);
    mma16(1);
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (q & 1) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
      if (((q + 1) * NR) / 16 != (q * NR) / 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  for (int kt = kb; kt < nk2; kt += 2) {
    step(std::false_type{}, kt);
    step(std::true_type{}, kt + 1);
  }

  // C tile (i, j): lane l holds row l%32, register r holds column 8(r/4) + 4(l/32) + r%4.
  const int hh = lane >> 5, l32 = lane & 31;
  // A whole tile of fp32 values (a partial, or an fp32 C without residual) at
  // dst[r * ld + c], 0 <= r, c < 256, 16-byte aligned rows: staged in LDS in two
  // halves of 128 rows (128 KB each, all of the slice buffers) and written one
  // 1 KB row per wave instruction. Written from the accumulator layout directly,
  // each instruction would touch 32 rows 16 bytes at a time (measured: 8192 x 8192
  // fp32 C at k = 1024, 241 -> 178 us). LDS rows: 64 16-byte chunks, chunk index
  // XOR row % 32, so both the accumulator-layout writes and the row reads hit
  // every bank once.
  auto store_tile_f32 = [&](float* dst, int64_t ld) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    auto quarter = [&](int qi) {  // 32 fp32 rows each
      return reinterpret_cast<float*>(qi == 0 ? As0 : qi == 1 ? As1 : qi == 2 ? Bs0 : Bs1);
    };
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      __syncthreads();  // the last slices (first half) or the previous half are consumed
      if (wm == half * 128) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float* lrow = quarter(i) + l32 * kBN;
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int chunk = (wn + 32 * j + 8 * q + 4 * hh) >> 2;
              *reinterpret_cast<f32x4*>(lrow + ((chunk ^ l32) << 2)) =
                  f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                        acc[i][j][4 * q + 3]};
            }
        }
      }
      __syncthreads();
#pragma unroll 4
      for (int it = 0; it < 32; ++it) {  // wave w writes rows 32 w .. +31 of the half
        const f32x4 x =
            *reinterpret_cast<const f32x4*>(quarter(w) + it * kBN + ((lane ^ it) << 2));
        *reinterpret_cast<f32x4*>(dst + (int64_t)(half * 128 + 32 * w + it) * ld + 4 * lane) = x;
      }
    }
  };
  if (partial && tail) {
    // a split tail's partial: tile-major [kpart][tail tile][256][256], whole tiles
    // (rows and columns past M, N hold sums of zeros and are never read back)
    store_tile_f32(part + ((int64_t)kpart * tail + (t_idx - head)) * kTileElems, kBN);
    return;
  }
  if (partial && (N & 3) == 0 && m0 + kBM <= M && n0 + kBN <= N) {
    // split-K partial of a whole tile
    store_tile_f32(part + (int64_t)blockIdx.y * M * N + (int64_t)m0 * N + n0, N);
    return;
  }
  if (partial) {
    // split-K partial: fp32 [M][N] slab of this k range, summed by splitk_reduce_kernel
    float* slab = part + (int64_t)blockIdx.y * M * N;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = m0 + wm + 32 * i + l32;
      if (row >= M) continue;
      float* prow = slab + (int64_t)row * N;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = n0 + wn + 32 * j + 8 * q + 4 * hh;
          if ((N & 3) == 0 && col + 3 < N) {
            typedef float f32x4 __attribute__((ext_vector_type(4)));
            *reinterpret_cast<f32x4*>(prow + col) =
                f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                      acc[i][j][4 * q + 3]};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (col + e < N) prow[col + e] = acc[i][j][4 * q + e];
          }
        }
    }
    return;
  }
  if constexpr (SMX) {
    // The wave's 128 columns of each row are one softmax group: lanes l and l + 32
    // hold 64 of them each. Max, then e = exp(logit - max) stored in TC and summed;
    // the target logit is picked by a select chain and stored by its lane.
    constexpr float kL2e = 1.4426950408889634f;
    const int cb = n0 + wn;  // first column of the group
    auto rows_of = [&](auto fullc) {
      constexpr bool FULL = decltype(fullc)::value;  // all 128 columns below N
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = m0 + wm + 32 * i + l32;
        const bool rv = row < M;
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int col = cb + 32 * j + 8 * (r >> 2) + 4 * hh + (r & 3);
            if (FULL || col < N) mx = fmaxf(mx, acc_read(acc[i][j][r]));
          }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        // reference point of the exponentials: an infinite max is replaced by 0
        const float ms = __builtin_isinf(mx) ? 0.f : mx * kL2e;
        // this lane's offset of the target column among its 64 (-1: not here)
        const int64_t tgt = rv ? smx.target[row] : -1;
        const int64_t toff = tgt - cb - 4 * hh;
        const int tk = (toff >= 0 && toff < 128 && (toff & 4) == 0 && tgt < N) ? (int)toff : -1;
        float sm = 0.f;
        TC* crow = C + (int64_t)(rv ? row : 0) * ldc;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int col = cb + 32 * j + 8 * q + 4 * hh;
            float ev[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float a = acc_read(acc[i][j][4 * q + e]);
              ev[e] = (FULL || col + e < N) ? __builtin_amdgcn_exp2f(__builtin_fmaf(a, kL2e, -ms))
                                            : 0.f;
              sm += ev[e];
            }
            if (rv) {
              if (vec_c && (FULL || col + 3 < N)) {
                typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
                auto bits = [](TC x) {
                  uint16_t u;
                  __builtin_memcpy(&u, &x, 2);
                  return (unsigned)u;
                };
                *reinterpret_cast<u32x2*>(crow + col) =
                    u32x2{bits(from_f32<TC>(ev[0])) | (bits(from_f32<TC>(ev[1])) << 16),
                          bits(from_f32<TC>(ev[2])) | (bits(from_f32<TC>(ev[3])) << 16)};
              } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  if (col + e < N) put<TC>(crow + col + e, ev[e]);
              }
            }
          }
        sm += __shfl_xor(sm, 32, 64);
        if (tk >= 0) {
          // acc[i][tk >> 5][4 ((tk >> 3) & 3) + (tk & 3)] by a select tree
          const int tj = tk >> 5, tq = (tk >> 3) & 3, te = tk & 3;
          float w4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v4[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int r = 4 * q + e;
              const float a0 = acc_read(acc[i][0][r]), a1 = acc_read(acc[i][1][r]);
              const float a2 = acc_read(acc[i][2][r]), a3 = acc_read(acc[i][3][r]);
              v4[q] = tj == 0 ? a0 : tj == 1 ? a1 : tj == 2 ? a2 : a3;
            }
            w4[e] = tq == 0 ? v4[0] : tq == 1 ? v4[1] : tq == 2 ? v4[2] : v4[3];
          }
          smx.tlogit[row] = te == 0 ? w4[0] : te == 1 ? w4[1] : te == 2 ? w4[2] : w4[3];
        }
        if (rv && hh == 0 && cb < N) {
          float* hs = smx.hstats + ((int64_t)row * smx.nh2 + (cb >> 7)) * 2;
          hs[0] = mx;
          hs[1] = sm;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (cb + 128 <= N) rows_of(std::true_type{});
    else rows_of(std::false_type{});
    return;
  }
  // C of the tile's segment (along M: rows; along N: columns)
  TC* cb = C;
  int64_t cshift = 0;
  if (SEG == 1) {
    const int sg = seg_of(seg, seg.dim == kSegM ? m0 : n0);
    if (seg.c[sg]) {
      cb = (TC*)seg.c[sg];
      cshift = seg.dim == kSegM ? (int64_t)seg.start[sg] * ldc : seg.start[sg];
    }
  }
  if constexpr (std::is_same<TC, float>::value) {
    if (!R && vec_c && m0 + kBM <= M && n0 + kBN <= N) {
      store_tile_f32(cb + ((int64_t)m0 * ldc - cshift) + n0, ldc);
      return;
    }
  } else {
    // A whole 16-bit tile is staged in LDS and written as whole 512-byte row
    // segments (16 bytes per lane, 2 rows per wave instruction): stored from the
    // accumulator layout directly, each instruction would touch 32 rows 16 bytes at
    // a time (8192 x 8192 at k = 1024: 187 -> 155 us). A residual is read and added
    // in the accumulator layout before the one rounding (R may be C: every lane has
    // read its elements of R before the barrier that precedes the row writes). LDS
    // rows: 32 16-byte chunks, chunk index XOR row % 32, so that both the
    // accumulator-layout writes and the row reads hit every bank once.
    if (vec_c && (ldc & 7) == 0 && m0 + kBM <= M && n0 + kBN <= N) {
      typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
      typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
      auto quarter = [&](int qi) {  // 64 tile rows each
        return qi == 0 ? As0 : qi == 1 ? As1 : qi == 2 ? Bs0 : Bs1;
      };
      auto bits = [](TC x) {
        uint16_t u;
        __builtin_memcpy(&u, &x, 2);
        return (unsigned)u;
      };
      __syncthreads();  // every wave is done with the last slices
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = wm + 32 * i + l32;
        uint16_t* lrow = quarter((wm >> 6) + (i >> 1)) + (r & 63) * kBN;
        const TC* rrow = R ? (const TC*)R + (int64_t)(m0 + r) * ldr : nullptr;
        const float* rrow32 = R ? (const float*)R + (int64_t)(m0 + r) * ldr : nullptr;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int chunk = (wn + 32 * j + 8 * q) >> 3;
            float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                          acc[i][j][4 * q + 3]};
            if (R) {
              const int col = n0 + wn + 32 * j + 8 * q + 4 * hh;
              float r4[4];
              if (r_f32) load_f32<float, 4>(rrow32 + col, r4);
              else load_f32<TC, 4>(rrow + col, r4);
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] += r4[e];
            }
            *reinterpret_cast<u32x2*>(lrow + ((chunk ^ (r & 31)) << 3) + 4 * hh) =
                u32x2{bits(from_f32<TC>(v[0])) | (bits(from_f32<TC>(v[1])) << 16),
                      bits(from_f32<TC>(v[2])) | (bits(from_f32<TC>(v[3])) << 16)};
          }
      }
      __syncthreads();
      const int chunk = lane & 31;
#pragma unroll 4
      for (int it = 0; it < 32; ++it) {
        const int r = 64 * w + 2 * it + hh;  // this wave's 64 rows: quarter w
        const u32x4 v = *reinterpret_cast<const u32x4*>(quarter(w) + (r & 63) * kBN +
                                                        ((chunk ^ (r & 31)) << 3));
        *reinterpret_cast<u32x4*>(cb + ((int64_t)(m0 + r) * ldc - cshift) + n0 + 8 * chunk) = v;
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = m0 + wm + 32 * i + l32;
    if (row >= M) continue;
    TC* crow = cb + ((int64_t)row * ldc - cshift);
    // residual row: of TC, or fp32 (r_f32: a running fp32 sum rounded into C)
    const TC* rrow = R ? (const TC*)R + (int64_t)row * ldr : nullptr;
    const float* rrow32 = R ? (const float*)R + (int64_t)row * ldr : nullptr;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = n0 + wn + 32 * j + 8 * q + 4 * hh;
        float v0 = acc[i][j][4 * q], v1 = acc[i][j][4 * q + 1];
        float v2 = acc[i][j][4 * q + 2], v3 = acc[i][j][4 * q + 3];
        if (rrow) {
          // C = R + A B: the residual (or, with R = C, the running sum) is read by
          // the lane that writes the same elements, and added in fp32.
          float r4[4] = {0.f, 0.f, 0.f, 0.f};
          if (vec_c && col + 3 < N) {
            if (r_f32) load_f32<float, 4>(rrow32 + col, r4);
            else load_f32<TC, 4>(rrow + col, r4);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (col + e < N) r4[e] = r_f32 ? rrow32[col + e] : to_f32(rrow[col + e]);
          }
          v0 += r4[0], v1 += r4[1], v2 += r4[2], v3 += r4[3];
        }
        if (vec_c && col + 3 < N) {
          if constexpr (std::is_same<TC, float>::value) {
            typedef float f32x4 __attribute__((ext_vector_type(4)));
            *reinterpret_cast<f32x4*>(crow + col) = f32x4{v0, v1, v2, v3};
          } else {
            typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
            auto bits = [](TC x) {
              uint16_t u;
              __builtin_memcpy(&u, &x, 2);
              return (unsigned)u;
            };
            *reinterpret_cast<u32x2*>(crow + col) =
                u32x2{bits(from_f32<TC>(v0)) | (bits(from_f32<TC>(v1)) << 16),
                      bits(from_f32<TC>(v2)) | (bits(from_f32<TC>(v3)) << 16)};
          }
        } else {
          if (col < N) put<TC>(crow + col, v0);
          if (col + 1 < N) put<TC>(crow + col + 1, v1);
          if (col + 2 < N) put<TC>(crow + col + 2, v2);
          if (col + 3 < N) put<TC>(crow + col + 3, v3);
        }
      }
  }
}

// fp32 operands (no fp32 MFMA path is worth its registers here): a plain tiled
// product, 64 x 64 outputs per 256-thread workgroup, 4 x 4 per thread, 16-deep
// k slices staged in LDS with every element bounds-checked. Used for fp32 inputs
// of the fused linear cross entropy.
template <bool AKC, bool BKC>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A,
                                                       const float* __restrict__ B,
                                                       float* C, int M, int N, int K,
                                                       int64_t lda, int64_t ldb, int64_t ldc,
                                                       int64_t a_rows, int64_t b_rows,
                                                       const float* R, int64_t ldr) {
  __shared__ float As[16][65], Bs[16][65];
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int e = threadIdx.x; e < 16 * 64; e += 256) {
      const int kk = e / 64, mm = e % 64;
      const int64_t k = k0 + kk, m = m0 + mm, n = n0 + mm;
      float av = 0.f, bv = 0.f;
      if (k < K && m < M) {
        const int64_t r = AKC ? m : k;
        if (r < a_rows) av = AKC ? A[m * lda + k] : A[k * lda + m];
      }
      if (k < K && n < N) {
        const int64_t r = BKC ? n : k;
        if (r < b_rows) bv = BKC ? B[n * ldb + k] : B[k * ldb + n];
      }
      As[kk][mm] = av;
      Bs[kk][mm] = bv;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += As[kk][ty * 4 + i] * Bs[kk][tx * 4 + j];
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
      if (m < M && n < N)
        C[(int64_t)m * ldc + n] = R ? acc[i][j] + R[(int64_t)m * ldr + n] : acc[i][j];
    }
}

// Split-K reduction: c[m][n] = r[m][n] + sum over s (in order) of part[s][m][n],
// rounded once to TC. Four consecutive columns per thread when N % 4 == 0.
template <typename TC, int V>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(
    const float* __restrict__ part, int splits, int M, int N, TC* C, int64_t ldc, const void* R,
    int64_t ldr, int r_f32, SegArgs seg) {
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
  const int64_t MN = (int64_t)M * N;
  if (idx >= MN) return;
  const int row = (int)(idx / N), col = (int)(idx - (int64_t)row * N);
  float v[V];
  load_f32<float, V>(part + idx, v);
  for (int s = 1; s < splits; ++s) {
    float w[V];
    load_f32<float, V>(part + s * MN + idx, w);
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] += w[e];
  }
  if (R) {
    float r[V];
    if (r_f32) load_f32<float, V>((const float*)R + (int64_t)row * ldr + col, r);
    else load_f32<TC, V>((const TC*)R + (int64_t)row * ldr + col, r);
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] += r[e];
  }
  store_f32<TC, V>(c_at(C, ldc, seg, row, col), v);
}

// The split tail's tiles: parts summed in order, the residual added, one rounding.
// Thread = 4 consecutive columns of one row of one tail tile.
template <typename TC>
__global__ __launch_bounds__(256) void splitk_tail_reduce_kernel(
    const float* __restrict__ part, int parts, int head, int tail, int tiles_m, int tiles, int M,
    int N, TC* C, int64_t ldc, const void* R, int64_t ldr, int r_f32, int vec_c, SegArgs seg) {
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (e >= (int64_t)tail * kTileElems) return;
  const int tt = (int)(e / kTileElems), rc = (int)(e % kTileElems);
  const int r = rc / kBN, c = rc % kBN;
  int tm, tn;
  tile_decode(head + tt, tiles_m, tiles, tm, tn);
  const int row = tm * kBM + r, col = tn * kBN + c;
  if (row >= M || col >= N) return;
  float v[4];
  load_f32<float, 4>(part + e, v);
  for (int p = 1; p < parts; ++p) {
    float w[4];
    load_f32<float, 4>(part + (int64_t)p * tail * kTileElems + e, w);
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] += w[q];
  }
  TC* cp = c_at(C, ldc, seg, row, col);  // 4 columns of one tile: one segment
  if (vec_c && col + 3 < N) {
    if (R) {
      float rr[4];
      if (r_f32) load_f32<float, 4>((const float*)R + (int64_t)row * ldr + col, rr);
      else load_f32<TC, 4>((const TC*)R + (int64_t)row * ldr + col, rr);
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] += rr[q];
    }
    store_f32<TC, 4>(cp, v);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (col + q >= N) break;
      float x = v[q];
      if (R) x += r_f32 ? ((const float*)R)[(int64_t)row * ldr + col + q]
                        : to_f32(((const TC*)R)[(int64_t)row * ldr + col + q]);
      put<TC>(cp + q, x);
    }
  }
}


// Explicit instantiation of one product kernel (KIND: `template` to define it in the
// including file, `extern template` to use one defined elsewhere). The kernels are
// instantiated across several sources (gemm_inst_*.hip) so that the build compiles
// them in parallel.
#define EG_GEMM_KERNEL(KIND, T, AKC, BKC, TC, SMX, SEG)                                      \
  KIND __global__ void gemm_kernel<T, AKC, BKC, TC, SMX, SEG>(                               \
      const uint16_t*, const uint16_t*, TC*, int, int, int, int64_t, int64_t, int64_t, int64_t, \
      int64_t, int, int, int, SmxArgs, const void*, int64_t, int, int, float*, int, int,       \
      SegArgs);
// The four layouts of one (operand, output, epilogue, segmentation) choice.
#define EG_GEMM_LAYOUTS(KIND, T, TC, SMX, SEG)            \
  EG_GEMM_KERNEL(KIND, T, true, true, TC, SMX, SEG)       \
  EG_GEMM_KERNEL(KIND, T, true, false, TC, SMX, SEG)      \
  EG_GEMM_KERNEL(KIND, T, false, true, TC, SMX, SEG)      \
  EG_GEMM_KERNEL(KIND, T, false, false, TC, SMX, SEG)
// Every product kernel the host code launches: plain products with 16-bit or fp32 C,
// segmented products (16-bit C), and the logits product with the softmax epilogue.
#define EG_GEMM_ALL_KERNELS(KIND, T)                       \
  EG_GEMM_LAYOUTS(KIND, T, T, false, 0)                    \
  EG_GEMM_LAYOUTS(KIND, T, float, false, 0)                \
  EG_GEMM_LAYOUTS(KIND, T, T, false, 1)                    \
  EG_GEMM_LAYOUTS(KIND, T, T, false, 2)                    \
  EG_GEMM_KERNEL(KIND, T, true, true, T, true, 0)

}  // namespace gk
}  // namespace eg
