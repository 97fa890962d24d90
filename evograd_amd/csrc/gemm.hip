// Host side of the dense products (eg_gemm, eg_gemm_segmented and the fused linear
// cross entropy's logits product): shape checks, split-K and split-tail planning,
// launches. The kernels are in gemm_kernel.hpp, instantiated by gemm_inst_*.hip.
#include "gemm_kernel.hpp"

namespace eg {
namespace gk {
// The product kernels are instantiated in the gemm_inst_*.hip sources, not here.
EG_GEMM_ALL_KERNELS(extern template, bf16_t)
EG_GEMM_ALL_KERNELS(extern template, f16_t)
}  // namespace gk
using namespace gk;

// Split-K: when the output has at most half as many tiles as kSplitTarget (one per
// CU of an MI355X; a constant, so the summation order depends on the shape only)
// and the caller's workspace holds the fp32 partials, K is cut into `splits` ranges
// of whole 64-deep slices, at least kMinSliceRun each.
constexpr int kSplitTarget = 256, kMaxSplits = 16, kMinSliceRun = 4;

int gemm_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  const int64_t nk = (K + kBK - 1) / kBK;
  if (tiles > kSplitTarget / 2) return 1;  // 128 tiles: 2 splits fill the 256 CUs
  int64_t s = std::min<int64_t>(kMaxSplits, kSplitTarget / tiles);
  s = std::min<int64_t>(s, nk / kMinSliceRun);
  if (s < 2) return 1;
  const int64_t per = (nk + s - 1) / s;
  return (int)((nk + per - 1) / per);
}

// Split tail: a product of more than one wave of tiles (kSplitTarget workgroups per
// wave) whose last wave is at most half full runs that wave's tiles in k parts,
// min(kMaxTailParts, kSplitTarget / tail, slices / kMinSliceRun) of them, so that the
// last wave fills the device (an 896-tile product: 3.5 waves -> 3 + 2 x 0.5); the
// parts' fp32 tiles are summed in order by splitk_tail_reduce_kernel. Shape-only.
constexpr int kMaxTailParts = 4;
struct TailPlan {
  int64_t head, tail;
  int parts, kt_per;
};
TailPlan gemm_tail(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
  const int64_t nk = (K + kBK - 1) / kBK;
  TailPlan p{tiles, 0, 1, 0};
  if (gemm_splits(M, N, K) > 1) return p;
  const int64_t waves = (tiles + kSplitTarget - 1) / kSplitTarget;
  const int64_t rem = tiles - (waves - 1) * kSplitTarget;
  if (waves < 2 || rem > kSplitTarget / 2) return p;
  const int64_t s = std::min<int64_t>({kMaxTailParts, kSplitTarget / rem, nk / kMinSliceRun});
  if (s < 2) return p;
  const int64_t per = (nk + s - 1) / s;
  p.head = tiles - rem;
  p.tail = rem;
  p.kt_per = (int)per;
  p.parts = (int)((nk + per - 1) / per);
  return p;
}

size_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int s = gemm_splits(M, N, K);
  if (s > 1) return (size_t)s * M * N * sizeof(float);
  const TailPlan p = gemm_tail(M, N, K);
  return p.tail ? (size_t)p.parts * p.tail * kTileElems * sizeof(float) : 0;
}

// C[M][N] = A B in fp32 accumulation; see the file comment for the layouts.
// a_kc: A is [a_rows][lda] holding rows m (else rows k); b_kc: B is [b_rows][ldb]
// holding rows n (else rows k). Rows at or past a_rows / b_rows read as zero.
namespace {
int gemm_impl(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
              int64_t lda, int64_t ldb, int64_t ldc, bool a_kc, bool b_kc, int64_t a_rows,
              int64_t b_rows, int dtype, int c_dtype, hipStream_t st, const char* name,
              const void* R, int64_t ldr, bool r_f32, void* ws, size_t ws_bytes,
              const SegArgs& seg);
}  // namespace

int gemm_launch(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                int64_t lda, int64_t ldb, int64_t ldc, bool a_kc, bool b_kc, int64_t a_rows,
                int64_t b_rows, int dtype, int c_dtype, hipStream_t st, const char* name,
                const void* R, int64_t ldr, bool r_f32, void* ws, size_t ws_bytes) {
  SegArgs none{};
  none.dim = kSegNone;
  return gemm_impl(A, B, C, M, N, K, lda, ldb, ldc, a_kc, b_kc, a_rows, b_rows, dtype, c_dtype, st,
                   name, R, ldr, r_f32, ws, ws_bytes, none);
}

namespace {
int gemm_impl(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
              int64_t lda, int64_t ldb, int64_t ldc, bool a_kc, bool b_kc, int64_t a_rows,
              int64_t b_rows, int dtype, int c_dtype, hipStream_t st, const char* name,
              const void* R, int64_t ldr, bool r_f32, void* ws, size_t ws_bytes,
              const SegArgs& seg) {
  if (M <= 0 || N <= 0) return 0;
  if (K <= 0) {
    set_error("%s: K must be positive", name);
    return 1;
  }
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff || a_rows < 0 || b_rows < 0) {
    set_error("%s: size out of range", name);
    return 1;
  }
  if (a_rows > (a_kc ? M : K) || b_rows > (b_kc ? N : K)) {
    set_error("%s: an operand holds more rows than the product reads", name);
    return 1;
  }
  if (R && r_f32 && c_dtype == EG_F32) r_f32 = false;  // the same thing
  if (dtype == EG_F32) {
    if (c_dtype != EG_F32) {
      set_error("%s: fp32 operands give an fp32 output", name);
      return 1;
    }
    if ((a_kc ? lda < K : lda < M) || (b_kc ? ldb < K : ldb < N) || ldc < N ||
        (R && ldr < N)) {
      set_error("%s: a leading dimension is smaller than its row", name);
      return 1;
    }
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    if (grid.y > 65535) {
      set_error("%s: M too large for the fp32 path", name);
      return 1;
    }
    auto go32 = [&](auto akc, auto bkc) {
      EG_LAUNCH((gemm_f32_kernel<decltype(akc)::value, decltype(bkc)::value>), grid, dim3(256),
                0, st, (const float*)A, (const float*)B, (float*)C, (int)M, (int)N, (int)K, lda,
                ldb, ldc, a_rows, b_rows, (const float*)R, ldr);
      return check_launch(name);
    };
    using TT = std::true_type;
    using FF = std::false_type;
    if (a_kc && b_kc) return go32(TT{}, TT{});
    if (a_kc) return go32(TT{}, FF{});
    if (b_kc) return go32(FF{}, TT{});
    return go32(FF{}, FF{});
  }
  if (dtype != EG_BF16 && dtype != EG_F16) {
    set_error("%s: operands must be fp32, bf16 or fp16", name);
    return 1;
  }
  if (c_dtype != EG_F32 && c_dtype != dtype) {
    set_error("%s: output must be fp32 or the operand dtype", name);
    return 1;
  }
  // A k-contiguous operand is read in whole 64-deep slices. With K % 64 != 0 that
  // reads its columns K .. roundup(K, 64): allowed when the row stride covers them
  // and the other operand is k-major (its rows past K read as zero, so those
  // columns, which must hold finite values, add nothing).
  const int64_t kpad = (K + kBK - 1) / kBK * kBK;
  const bool k_ok = (!a_kc && !b_kc) || K % kBK == 0 ||
                    (a_kc != b_kc && (a_kc ? lda : ldb) >= kpad);
  if (!k_ok || lda % 8 || ldb % 8 || !aligned16(A) || !aligned16(B)) {
    set_error("%s: K-contiguous operands need K %% 64 == 0 (or, against a k-major operand, a "
              "row stride of at least K rounded up to 64); strides must be multiples of 8 "
              "elements and bases 16-byte aligned", name);
    return 1;
  }
  // Row widths: a column-segmented operand's rows are one segment wide.
  int64_t seg_max = 0;
  for (int i = 0; seg.dim != kSegNone && i < seg.n; ++i)
    seg_max = std::max<int64_t>(seg_max, seg.start[i + 1] - seg.start[i]);
  const bool a_cols = (seg.dim == kSegK && a_kc) || (seg.dim == kSegM && !a_kc);
  const bool b_cols = (seg.dim == kSegK && b_kc) || (seg.dim == kSegN && !b_kc);
  const bool c_cols = seg.dim == kSegN && seg.c[0];
  const int64_t a_w = a_cols && seg.a[0] ? seg_max : (a_kc ? K : M);
  const int64_t b_w = b_cols && seg.b[0] ? seg_max : (b_kc ? K : N);
  const int64_t c_w = c_cols ? seg_max : N;
  if (lda < a_w || ldb < b_w || ldc < c_w || (R && ldr < N)) {
    set_error("%s: a leading dimension is smaller than its row", name);
    return 1;
  }
  // Per-lane byte offsets inside one slice are 32-bit: up to 255 rows (K-contiguous)
  // or 63 rows (K-major) of the stride.
  if ((a_kc ? 256 : 64) * lda * 2 >= ((int64_t)1 << 31) ||
      (b_kc ? 256 : 64) * ldb * 2 >= ((int64_t)1 << 31)) {
    set_error("%s: row stride too large", name);
    return 1;
  }
  const int64_t tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  const int64_t tiles = tiles_m * tiles_n;
  if (tiles > 0x7fffffff / 2) {
    set_error("%s: too many tiles", name);
    return 1;
  }
  const unsigned grid = (unsigned)(((tiles + 7) / 8) * 8);
  // 16-byte (fp32) or 8-byte (16-bit) row pieces of C need ldc % 4 == 0 and a
  // 16-byte aligned base; otherwise the kernel stores element by element.
  const int vec_c = (ldc % 4 == 0) && aligned16(C) &&
                    (!R || ((ldr % 4 == 0) && aligned16(R)));
  const bool ws_ok = ws && aligned16(ws) && ws_bytes >= gemm_workspace_bytes(M, N, K);
  int splits = gemm_splits(M, N, K);
  if (splits > 1 && !ws_ok) splits = 1;
  TailPlan tp = gemm_tail(M, N, K);
  if (!ws_ok) tp = TailPlan{tiles, 0, 1, 0};
  const int nk = (int)((K + kBK - 1) / kBK);
  const int kt_per = tp.tail ? tp.kt_per : (nk + splits - 1) / splits;
  const unsigned grid_x = tp.tail ? (unsigned)(tp.head + tp.tail * tp.parts) : grid;
  auto go = [&](auto tag, auto ctag, auto akc, auto bkc) {
    using T = decltype(tag);
    using TC = decltype(ctag);
    constexpr bool AK = decltype(akc)::value, BK = decltype(bkc)::value;
    float* part = (splits > 1 || tp.tail) ? (float*)ws : nullptr;
    if (seg.dim != kSegNone) {
      // segmented products: 16-bit C only (one more instantiation per layout)
      if constexpr (std::is_same<T, TC>::value) {
        if (seg.dim == kSegK)
          EG_LAUNCH((gemm_kernel<T, AK, BK, TC, false, 2>), dim3(grid_x, (unsigned)splits),
                    dim3(kThreads), 0, st, (const uint16_t*)A, (const uint16_t*)B, (TC*)C, (int)M,
                    (int)N, (int)K, lda, ldb, ldc, a_rows, b_rows, (int)tiles_m, (int)tiles, vec_c,
                    SmxArgs{}, R, ldr, (int)r_f32, kt_per, part, (int)tp.head, (int)tp.tail, seg);
        else
          EG_LAUNCH((gemm_kernel<T, AK, BK, TC, false, 1>), dim3(grid_x, (unsigned)splits),
                    dim3(kThreads), 0, st, (const uint16_t*)A, (const uint16_t*)B, (TC*)C, (int)M,
                    (int)N, (int)K, lda, ldb, ldc, a_rows, b_rows, (int)tiles_m, (int)tiles, vec_c,
                    SmxArgs{}, R, ldr, (int)r_f32, kt_per, part, (int)tp.head, (int)tp.tail, seg);
      } else {
        set_error("%s: segmented products write C in the operands' dtype", name);
        return 1;
      }
    } else {
      EG_LAUNCH((gemm_kernel<T, AK, BK, TC>), dim3(grid_x, (unsigned)splits), dim3(kThreads), 0,
                st, (const uint16_t*)A, (const uint16_t*)B, (TC*)C, (int)M, (int)N, (int)K, lda,
                ldb, ldc, a_rows, b_rows, (int)tiles_m, (int)tiles, vec_c, SmxArgs{}, R, ldr,
                (int)r_f32, kt_per, part, (int)tp.head, (int)tp.tail, seg);
    }
    if (int e = check_launch(name)) return e;
    if (tp.tail) {
      EG_LAUNCH((splitk_tail_reduce_kernel<TC>), dim3((unsigned)(tp.tail * (kTileElems / 1024))),
                dim3(256), 0, st, (const float*)part, tp.parts, (int)tp.head, (int)tp.tail,
                (int)tiles_m, (int)tiles, (int)M, (int)N, (TC*)C, ldc, R, ldr, (int)r_f32, vec_c,
                seg);
      return check_launch(name);
    }
    if (splits == 1) return 0;
    const bool v4 = (N % 4 == 0) && vec_c;
    const int64_t n = M * N / (v4 ? 4 : 1);
    const unsigned rg = (unsigned)((n + 255) / 256);
    if (v4)
      EG_LAUNCH((splitk_reduce_kernel<TC, 4>), dim3(rg), dim3(256), 0, st, part, splits, (int)M,
                (int)N, (TC*)C, ldc, R, ldr, (int)r_f32, seg);
    else
      EG_LAUNCH((splitk_reduce_kernel<TC, 1>), dim3(rg), dim3(256), 0, st, part, splits, (int)M,
                (int)N, (TC*)C, ldc, R, ldr, (int)r_f32, seg);
    return check_launch(name);
  };
  auto layouts = [&](auto tag, auto ctag) {
    using TT = std::true_type;
    using FF = std::false_type;
    if (a_kc && b_kc) return go(tag, ctag, TT{}, TT{});
    if (a_kc) return go(tag, ctag, TT{}, FF{});
    if (b_kc) return go(tag, ctag, FF{}, TT{});
    return go(tag, ctag, FF{}, FF{});
  };
  if (dtype == EG_BF16)
    return c_dtype == EG_F32 ? layouts(bf16_t{}, float{}) : layouts(bf16_t{}, bf16_t{});
  return c_dtype == EG_F32 ? layouts(f16_t{}, float{}) : layouts(f16_t{}, f16_t{});
}
}  // namespace

int64_t flce_groups(int64_t n) { return 2 * ((n + kBN - 1) / kBN); }

int gemm_logits_softmax_launch(const void* x, const void* w, void* e, int64_t M, int64_t N,
                               int64_t K, int64_t ldx, int64_t ldw, int64_t lde,
                               const int64_t* target, float* hstats, float* tlogit, int dtype,
                               hipStream_t st, const char* name) {
  if (M <= 0 || N <= 0) return 0;
  if (dtype != EG_BF16 && dtype != EG_F16) {
    set_error("%s: the softmax epilogue takes bf16 or fp16 operands", name);
    return 1;
  }
  if (K <= 0 || K % kBK || ldx % 8 || ldw % 8 || ldx < K || ldw < K || lde < N ||
      !aligned16(x) || !aligned16(w)) {
    set_error("%s: logits product needs K %% 64 == 0, strides >= K in multiples of 8 and "
              "16-byte aligned operands", name);
    return 1;
  }
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff || 256 * ldx * 2 >= ((int64_t)1 << 31) ||
      256 * ldw * 2 >= ((int64_t)1 << 31)) {
    set_error("%s: size out of range", name);
    return 1;
  }
  const int64_t tiles_m = (M + kBM - 1) / kBM, tiles_n = (N + kBN - 1) / kBN;
  const int64_t tiles = tiles_m * tiles_n;
  if (tiles > 0x7fffffff / 2 || flce_groups(N) > 0x7fffffff) {
    set_error("%s: too many tiles", name);
    return 1;
  }
  const unsigned grid = (unsigned)(((tiles + 7) / 8) * 8);
  const int vec_c = (lde % 4 == 0) && aligned16(e);
  const SmxArgs smx{target, hstats, tlogit, (int)flce_groups(N)};
  auto go = [&](auto tag) {
    using T = decltype(tag);
    EG_LAUNCH((gemm_kernel<T, true, true, T, true>), dim3(grid), dim3(kThreads), 0, st,
              (const uint16_t*)x, (const uint16_t*)w, (T*)e, (int)M, (int)N, (int)K, ldx, ldw,
              lde, M, N, (int)tiles_m, (int)tiles, vec_c, smx, (const void*)nullptr, (int64_t)0,
              0, 0, (float*)nullptr, (int)tiles, 0, SegArgs{});
    return check_launch(name);
  };
  return dtype == EG_BF16 ? go(bf16_t{}) : go(f16_t{});
}

}  // namespace eg

using namespace eg;

extern "C" size_t eg_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int dtype) {
  if (dtype != EG_BF16 && dtype != EG_F16) return 0;
  return gemm_workspace_bytes(m, n, k);
}

extern "C" int eg_gemm(const void* a, const void* b, void* c, const void* r, int64_t m,
                       int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int64_t ldr,
                       int a_k_contiguous, int b_k_contiguous, int dtype, int c_dtype,
                       void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (m < 0 || n < 0 || k < 0) {
    set_error("eg_gemm: negative size");
    return 1;
  }
  if (m > 0 && n > 0 && (!a || !b || !c)) {
    set_error("eg_gemm: null pointer");
    return 1;
  }
  const bool akc = a_k_contiguous != 0, bkc = b_k_contiguous != 0;
  return gemm_launch(a, b, c, m, n, k, lda, ldb, ldc, akc, bkc, akc ? m : k, bkc ? n : k, dtype,
                     c_dtype, as_stream(stream), "eg_gemm", r, ldr, false, workspace,
                     workspace_bytes);
}

extern "C" int eg_gemm_segmented(const void* a, const void* b, void* c, int64_t m, int64_t n,
                                 int64_t k, int64_t lda, int64_t ldb, int64_t ldc,
                                 int a_k_contiguous, int b_k_contiguous, int seg_dim, int nseg,
                                 const int64_t* seg_sizes, const void* const* a_segs,
                                 const void* const* b_segs, void* const* c_segs, int dtype,
                                 int c_dtype, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  clear_error();
  const char* name = "eg_gemm_segmented";
  if (m < 0 || n < 0 || k < 0) {
    set_error("%s: negative size", name);
    return 1;
  }
  if (seg_dim < kSegM || seg_dim > kSegK || nseg < 1 || nseg > kMaxSegs || !seg_sizes) {
    set_error("%s: seg_dim must be 1 (M), 2 (N) or 3 (K), with 1 to %d segment sizes", name,
              kMaxSegs);
    return 1;
  }
  if (dtype != EG_BF16 && dtype != EG_F16) {
    set_error("%s: operands must be bf16 or fp16", name);
    return 1;
  }
  // the operands the segmented dimension indexes: M -> A, C; N -> B, C; K -> A, B
  const bool a_ok = seg_dim != kSegN, b_ok = seg_dim != kSegM, c_ok = seg_dim != kSegK;
  if ((a_segs && !a_ok) || (b_segs && !b_ok) || (c_segs && !c_ok) ||
      (!a_segs && !b_segs && !c_segs)) {
    set_error("%s: segment pointers given for an operand the dimension does not index, or "
              "for none", name);
    return 1;
  }
  const bool akc = a_k_contiguous != 0, bkc = b_k_contiguous != 0;
  const int64_t extent = seg_dim == kSegM ? m : seg_dim == kSegN ? n : k;
  const int64_t unit = seg_dim == kSegK ? kBK : kBM;
  SegArgs g{};
  g.dim = seg_dim;
  g.n = nseg;
  int64_t at = 0;
  for (int i = 0; i < nseg; ++i) {
    if (seg_sizes[i] <= 0 || (i + 1 < nseg && seg_sizes[i] % unit)) {
      set_error("%s: segment sizes must be positive and, except the last, multiples of %lld",
                name, (long long)unit);
      return 1;
    }
    g.start[i] = (int)at;
    at += seg_sizes[i];
    if (at > 0x7fffffff) {
      set_error("%s: size out of range", name);
      return 1;
    }
  }
  for (int i = nseg; i <= kMaxSegs; ++i) g.start[i] = (int)at;
  if (at != extent) {
    set_error("%s: segment sizes add up to %lld, the segmented dimension is %lld", name,
              (long long)at, (long long)extent);
    return 1;
  }
  if (seg_dim == kSegK && (akc || bkc) && k % kBK) {
    set_error("%s: segments along K with a k-contiguous operand need K %% 64 == 0", name);
    return 1;
  }
  for (int i = 0; i < nseg; ++i) {
    g.a[i] = a_segs ? a_segs[i] : nullptr;
    g.b[i] = b_segs ? b_segs[i] : nullptr;
    g.c[i] = c_segs ? c_segs[i] : nullptr;
    if ((a_segs && !g.a[i]) || (b_segs && !g.b[i]) || (c_segs && !g.c[i])) {
      set_error("%s: null segment pointer", name);
      return 1;
    }
    if ((g.a[i] && !aligned16(g.a[i])) || (g.b[i] && !aligned16(g.b[i])) ||
        (g.c[i] && !aligned16(g.c[i]))) {
      set_error("%s: segment pointers must be 16-byte aligned", name);
      return 1;
    }
  }
  // a segmented operand's plain pointer stands for its first segment
  const void* pa = a_segs ? a_segs[0] : a;
  const void* pb = b_segs ? b_segs[0] : b;
  void* pc = c_segs ? c_segs[0] : c;
  if (m > 0 && n > 0 && (!pa || !pb || !pc)) {
    set_error("%s: null pointer", name);
    return 1;
  }
  if (m == 0 || n == 0) return 0;
  return gemm_impl(pa, pb, pc, m, n, k, lda, ldb, ldc, akc, bkc, akc ? m : k, bkc ? n : k, dtype,
                   c_dtype, as_stream(stream), name, nullptr, 0, false, workspace,
                   workspace_bytes, g);
}
