// Shared device helpers for the gfx950 kernels: dtype conversion with
// round-to-nearest-even (the rounding torch's .to(dtype) uses), 16-byte vector
// memory access, wave64 and workgroup reductions with a fixed combine order,
// and the thread-local error slot behind eg_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/evograd_hip.h"

namespace eg {

constexpr int kWave = 64;  // CDNA wavefront width

// ------------------------------------------------------------------ errors
void set_error(const char* fmt, ...);
// Called first by every entry point: clears the error slot and starts a new
// call for the kernel-timing hook (eg_time_kernel).
void clear_error();
// Turns a failed launch into an error return; reads (and clears) the HIP
// runtime's sticky launch error.
int check_launch(const char* what);

// ------------------------------------------------------------ dtype tags
struct bf16_t { uint16_t bits; };
typedef _Float16 f16_t;

template <typename T> struct DT;
template <> struct DT<float>  { static constexpr int id = EG_F32; };
template <> struct DT<f16_t>  { static constexpr int id = EG_F16; };
template <> struct DT<bf16_t> { static constexpr int id = EG_BF16; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16_t v) { return (float)v; }
__device__ __forceinline__ float to_f32(bf16_t v) {
  return __uint_as_float(((uint32_t)v.bits) << 16);
}

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950); NaN
// stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  const __bf16 b = (__bf16)f;
  uint16_t u;
  __builtin_memcpy(&u, &b, 2);
  return u;
}

// Two fp32 values -> packed pair of 16-bit values (one v_cvt_pk_* instruction),
// round to nearest even; `lo` lands in bits 0..15.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t r = __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t);
  uint32_t u;
  __builtin_memcpy(&u, &r, 4);
  return u;
}
__device__ __forceinline__ uint32_t pack2_f16(float lo, float hi) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  const f16x2_t r = __builtin_convertvector((f32x2_t){lo, hi}, f16x2_t);
  uint32_t u;
  __builtin_memcpy(&u, &r, 4);
  return u;
}

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float v) { return (f16_t)v; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) {
  bf16_t r; r.bits = f32_to_bf16_bits(v); return r;
}

// Round an fp32 value to T and widen it back (the value a .to(T) would hold).
template <typename T> __device__ __forceinline__ float round_to(float v) {
  return to_f32(from_f32<T>(v));
}

// ------------------------------------------------------- vector memory access
// VEC elements of T packed into one naturally aligned load/store (16 bytes when
// VEC * sizeof(T) == 16, which the hot paths use: global_load_dwordx4).
template <typename T, int VEC>
struct alignas(sizeof(T) * VEC) Pack {
  T v[VEC];
};

template <typename T, int VEC>
__device__ __forceinline__ void load_f32(const T* __restrict__ p, float (&out)[VEC]) {
  Pack<T, VEC> pk = *reinterpret_cast<const Pack<T, VEC>*>(p);
#pragma unroll
  for (int i = 0; i < VEC; ++i) out[i] = to_f32(pk.v[i]);
}

template <typename T, int VEC>
__device__ __forceinline__ void store_f32(T* __restrict__ p, const float (&in)[VEC]) {
  Pack<T, VEC> pk;
#pragma unroll
  for (int i = 0; i < VEC; ++i) pk.v[i] = from_f32<T>(in[i]);
  *reinterpret_cast<Pack<T, VEC>*>(p) = pk;
}

// Streaming variants: data touched once per kernel; the non-temporal hint keeps
// it from displacing reused lines (tables, weights) in L2.
template <typename T, int VEC>
__device__ __forceinline__ void load_f32_nt(const T* __restrict__ p, float (&out)[VEC]) {
  static_assert(sizeof(T) * VEC == 16, "nt path is for 16-byte packs");
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  Pack<T, VEC> pk;
  __builtin_memcpy(&pk, &raw, 16);
#pragma unroll
  for (int i = 0; i < VEC; ++i) out[i] = to_f32(pk.v[i]);
}

template <typename T, int VEC>
__device__ __forceinline__ void store_f32_nt(T* __restrict__ p, const float (&in)[VEC]) {
  static_assert(sizeof(T) * VEC == 16, "nt path is for 16-byte packs");
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  Pack<T, VEC> pk;
#pragma unroll
  for (int i = 0; i < VEC; ++i) pk.v[i] = from_f32<T>(in[i]);
  u32x4 raw;
  __builtin_memcpy(&raw, &pk, 16);
  __builtin_nontemporal_store(raw, reinterpret_cast<u32x4*>(p));
}

// Streaming when NT and the pack is 16 bytes, plain otherwise.
template <typename T, int VEC, bool NT>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, float (&out)[VEC]) {
  if constexpr (NT && sizeof(T) * VEC == 16) load_f32_nt<T, VEC>(p, out);
  else load_f32<T, VEC>(p, out);
}
template <typename T, int VEC, bool NT>
__device__ __forceinline__ void store_vec(T* __restrict__ p, const float (&in)[VEC]) {
  if constexpr (NT && sizeof(T) * VEC == 16) store_f32_nt<T, VEC>(p, in);
  else store_f32<T, VEC>(p, in);
}

// ------------------------------------------------------------- reductions
struct SumOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
  static __device__ __forceinline__ float identity() { return 0.f; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
  static __device__ __forceinline__ float identity() { return -INFINITY; }
};

// Butterfly over the 64 lanes; every lane ends with the same value, combined in
// the same order on every run.
template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
#pragma unroll
  for (int off = kWave / 2; off >= 1; off >>= 1) v = op(v, __shfl_xor(v, off, kWave));
  return v;
}

// Workgroup reduction of BLOCK threads. `lds` must hold BLOCK/64 floats. The
// per-wave results are combined in wave order, so the result is bit-identical
// across runs. Ends with every thread holding the result; callers that reuse
// `lds` must __syncthreads() first (done here at entry).
template <int BLOCK, typename Op>
__device__ __forceinline__ float block_reduce(float v, Op op, float* lds) {
  constexpr int NW = BLOCK / kWave;
  v = wave_reduce(v, op);
  if constexpr (NW == 1) {
    return v;
  } else {
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    __syncthreads();
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    float r = lds[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) r = op(r, lds[w]);
    return r;
  }
}

// Two sums at once (one barrier pair instead of two); used by the norm backwards.
template <int BLOCK>
__device__ __forceinline__ void block_reduce2(float& a, float& b, float* lds) {
  constexpr int NW = BLOCK / kWave;
  a = wave_reduce(a, SumOp());
  b = wave_reduce(b, SumOp());
  if constexpr (NW > 1) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = threadIdx.x / kWave;
    __syncthreads();
    if (lane == 0) { lds[wid] = a; lds[NW + wid] = b; }
    __syncthreads();
    float ra = lds[0], rb = lds[NW];
#pragma unroll
    for (int w = 1; w < NW; ++w) { ra += lds[w]; rb += lds[NW + w]; }
    a = ra; b = rb;
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Bounded buffer accesses on gfx950 (relied on by the kernels that use them):
//  - a buffer load whose offset lies outside the resource's range returns zero;
//  - a buffer->LDS load (buffer_load ... lds) outside the range writes zero into
//    the lane's LDS slot, exactly as the register load returns zero (the products'
//    ragged-k and odd-slice-count cases in tests/test_gpu_gemm.py hold only if it
//    does);
//  - a buffer store outside the range is dropped.

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------ launching
// True when this launch is the one eg_time_kernel armed for the current call;
// then *start / *stop are the events to record around it.
bool timed_launch(hipEvent_t* start, hipEvent_t* stop);
// Records the kernel expression of the timed launch (its name is kept for
// eg_time_kernel_label).
void set_timed_label(const char* kernel_expr);

// Every kernel is launched through EG_LAUNCH: a plain launch, or, for the launch
// armed by eg_time_kernel, hipExtLaunchKernelGGL with the caller's events, which
// the dispatch itself records at the kernel's start and end.
#define EG_LAUNCH(KERNEL, GRID, BLOCK, SHMEM, STREAM, ...)                              \
  do {                                                                                \
    hipEvent_t eg_t0_ = nullptr, eg_t1_ = nullptr;                                    \
    if (::eg::timed_launch(&eg_t0_, &eg_t1_)) {                                       \
      ::eg::set_timed_label(#KERNEL);                                                 \
      hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, SHMEM, STREAM, eg_t0_, eg_t1_, 0,     \
                            __VA_ARGS__);                                             \
    } else                                                                            \
      hipLaunchKernelGGL(KERNEL, GRID, BLOCK, SHMEM, STREAM, __VA_ARGS__);            \
  } while (0)

// Zeroes `bytes` bytes with a small kernel (no hipMemsetAsync, so the call is
// safe inside a captured graph). Returns 0 or an error code.
int zero_fill(void* p, size_t bytes, hipStream_t st, const char* what);

// The MFMA product behind eg_gemm (gemm_kernel.hpp, launched by gemm.hip): c[m][n] = sum_k a(m, k) b(k, n) with
// fp32 accumulation. a_kc: a is [a_rows][lda] holding rows m, else rows k; b_kc:
// b is [b_rows][ldb] holding rows n, else rows k; rows at or past a_rows / b_rows
// read as zero. bf16/fp16 operands need k % 64 == 0 for a k-contiguous operand.
// With r non-null the output is c = r + a b (r of c_dtype, or fp32 with r_f32; row
// stride ldr; added in fp32 before c is rounded); r == c with ldr == ldc
// accumulates in place. With a workspace of at least gemm_workspace_bytes(m, n, k)
// a product of few output tiles splits k (fp32 partials, a fixed-order sum).
size_t gemm_workspace_bytes(int64_t m, int64_t n, int64_t k);
int gemm_launch(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
                int64_t lda, int64_t ldb, int64_t ldc, bool a_kc, bool b_kc, int64_t a_rows,
                int64_t b_rows, int dtype, int c_dtype, hipStream_t st, const char* name,
                const void* r = nullptr, int64_t ldr = 0, bool r_f32 = false,
                void* ws = nullptr, size_t ws_bytes = 0);

// The logits product of the fused linear cross entropy with its softmax terms
// formed in the epilogue (gemm_kernel.hpp), 16-bit operands only: for logits = x w^T
// (x [m][ldx] and w [n][ldw] both k-contiguous, k % 64 == 0) it writes, per
// 128-column group h of a row (columns 128h .. 128h + 127),
//   e[row][col] = exp(logit - mx_h) in the operand dtype (ld lde),
//   hstats[(row * nh2 + h) * 2 + {0, 1}] = mx_h, sum over the group of exp(logit - mx_h),
// with nh2 = flce_groups(n), and tlogit[row] = logit[row][target[row]] (fp32) when
// the target is a column of [0, n); nothing for rows whose target is not.
int64_t flce_groups(int64_t n);
int gemm_logits_softmax_launch(const void* x, const void* w, void* e, int64_t m, int64_t n,
                               int64_t k, int64_t ldx, int64_t ldw, int64_t lde,
                               const int64_t* target, float* hstats, float* tlogit, int dtype,
                               hipStream_t st, const char* name);

// Causal GQA attention on plain fp32 arithmetic (attn_generic.hip) for the shapes
// the MFMA kernels do not take: any dtype, even head_dim <= 128. Arguments as
// eg_attn_gqa_fwd / eg_attn_gqa_bwd, already validated; delta is the backward's
// fp32 [B, H, S] workspace. With tables rc, rs (fp32 [S, D]) the forward rotates q
// as it loads it (k already rotated) and the backward takes the rotated q, k and
// writes dq, dk for the pre-rotation ones.
int attn_generic_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B,
                     int64_t H, int64_t Hkv, int64_t S, int64_t D, float scale, int dtype,
                     hipStream_t st, const float* rc = nullptr, const float* rs = nullptr);
int attn_generic_bwd(const void* dout, const void* q, const void* k, const void* v,
                     const void* o, const float* lse, void* dq, void* dk, void* dv, float* delta,
                     int64_t B, int64_t H, int64_t Hkv, int64_t S, int64_t D, float scale,
                     int dtype, hipStream_t st, const float* rc = nullptr,
                     const float* rs = nullptr);

// The RoPE launch behind eg_rope (rope.hip), for entry points that rotate as one
// step of a longer launch sequence: arguments as eg_rope's, already validated.
int rope_apply(const void* q, const void* k, void* q_out, void* k_out, const void* cos,
               const void* sin, int64_t batch, int64_t heads_q, int64_t heads_k,
               int64_t tokens, int64_t head_dim, int dtype, int table_dtype, bool inverse,
               hipStream_t st);


}  // namespace eg

// Dispatch on the runtime dtype tag; `FN` is a generic lambda taking a T* tag.
#define EG_DISPATCH_FLOAT(dtype, name, ...)                                      \
  [&]() -> int {                                                                 \
    switch (dtype) {                                                             \
      case EG_F32: { using scalar_t = float; return __VA_ARGS__(); }             \
      case EG_F16: { using scalar_t = eg::f16_t; return __VA_ARGS__(); }         \
      case EG_BF16: { using scalar_t = eg::bf16_t; return __VA_ARGS__(); }       \
      default: eg::set_error("%s: unsupported dtype %d", name, (int)(dtype));    \
               return 1;                                                         \
    }                                                                            \
  }()
