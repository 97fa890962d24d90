// Half-rotated RoPE forward/backward for gfx950, q and k in one launch.
//
// Follows rope_forward_ref (src/evograd/ops/level1/rope/forward_ref.py:28-47):
//   y = x * cos + rotate_half(x) * sin, rotate_half(x) = [-x2, x1]
// evaluated in fp32 and cast back. The backward declared at
// src/evograd/ops/level1/rope/__init__.py:124-130 is the transpose rotation,
//   dx = dy * cos + [dy2, -dy1] * sin,
// which is this kernel with the sine negated (`inverse`).
//
// Layout: x [batch, heads, tokens, head_dim] row-major; cos/sin [tokens, head_dim].
// A thread owns one (token, chunk) pair, chunk = VEC consecutive lanes of the
// first half plus the matching VEC lanes of the second half. It serves a group of
// four heads of one batch entry with one load of its four table slices, so the
// tables cost one read per (batch, head group) instead of one per row; the x
// traffic is pure 16-byte streaming, all of a group's loads issued before its
// first store.
#include "eg_common.hpp"

namespace eg {
namespace {

constexpr int kRopeBlock = 256;
// Heads per group: enough groups to fill the chip, few enough to amortise the
// table loads over several rows.
constexpr int kHeadsPerGroup = 4;

template <typename T, typename TT, int VEC, bool NT>
__global__ __launch_bounds__(kRopeBlock) void rope_kernel(
    const T* __restrict__ q, const T* __restrict__ k, T* __restrict__ qo, T* __restrict__ ko,
    const TT* __restrict__ cosv, const TT* __restrict__ sinv, int heads_q, int heads_k,
    int tokens, int head_dim, int groups_q, int groups_k, float sgn) {
  constexpr int HPG = kHeadsPerGroup;
  const int half = head_dim >> 1;
  const int cpr = half / VEC;  // chunks per row
  const int64_t idx = (int64_t)blockIdx.x * kRopeBlock + threadIdx.x;
  const int t = (int)(idx / cpr);
  if (t >= tokens) return;
  const int ch = (int)(idx - (int64_t)t * cpr);
  const int groups = groups_q + groups_k;
  const int b = blockIdx.y / groups;
  const int g = blockIdx.y - b * groups;
  const bool isq = g < groups_q;
  const T* __restrict__ src = isq ? q : k;
  T* __restrict__ dst = isq ? qo : ko;
  const int heads = isq ? heads_q : heads_k;
  const int h0 = (isq ? g : g - groups_q) * HPG;
  const int nh = min(HPG, heads - h0);

  const int64_t toff = (int64_t)t * head_dim + ch * VEC;
  const int64_t row_stride = (int64_t)tokens * head_dim;
  const int64_t off0 = ((int64_t)b * heads + h0) * row_stride + toff;
  float c1[VEC], c2[VEC], s1[VEC], s2[VEC];
  auto load_tables = [&] {
    load_f32<TT, VEC>(cosv + toff, c1);
    load_f32<TT, VEC>(cosv + toff + half, c2);
    load_f32<TT, VEC>(sinv + toff, s1);
    load_f32<TT, VEC>(sinv + toff + half, s2);
#pragma unroll
    for (int i = 0; i < VEC; ++i) { s1[i] *= -sgn; s2[i] *= sgn; }
  };
  auto rotate = [&](const float* x1, const float* x2, int64_t off) {
    float y1[VEC], y2[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      y1[i] = x1[i] * c1[i] + x2[i] * s1[i];
      y2[i] = x2[i] * c2[i] + x1[i] * s2[i];
    }
    store_vec<T, VEC, NT>(dst + off, y1);
    store_vec<T, VEC, NT>(dst + off + half, y2);
  };
  if (nh == HPG) {
    // A full group: every row's loads, then the tables, are issued before the
    // first store (the scheduling barrier keeps the compiler from interleaving
    // them again; 119.8 -> 114.5 us at q [8, 32, 4096, 128] + k [8, 8, 4096, 128]).
    float x1[HPG][VEC], x2[HPG][VEC];
#pragma unroll
    for (int j = 0; j < HPG; ++j) {
      load_vec<T, VEC, NT>(src + off0 + j * row_stride, x1[j]);
      load_vec<T, VEC, NT>(src + off0 + j * row_stride + half, x2[j]);
    }
    load_tables();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < HPG; ++j) rotate(x1[j], x2[j], off0 + j * row_stride);
  } else {
    load_tables();
    for (int j = 0; j < nh; ++j) {
      float x1[VEC], x2[VEC];
      load_vec<T, VEC, NT>(src + off0 + j * row_stride, x1);
      load_vec<T, VEC, NT>(src + off0 + j * row_stride + half, x2);
      rotate(x1, x2, off0 + j * row_stride);
    }
  }
}

inline bool aligned_to(const void* p, size_t n) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) % n) == 0;
}

template <typename T, typename TT, int VEC>
int launch_rope(const void* q, const void* k, void* qo, void* ko, const void* cosv,
                const void* sinv, int64_t batch, int64_t hq, int64_t hk, int64_t tokens,
                int64_t head_dim, float sgn, hipStream_t st) {
  const int hpg = kHeadsPerGroup;
  const int gq = (int)((hq + hpg - 1) / hpg);
  const int gk = (int)((hk + hpg - 1) / hpg);
  const int64_t gy = batch * (gq + gk);
  const int64_t threads = tokens * (head_dim / 2 / VEC);
  const int64_t gx = (threads + kRopeBlock - 1) / kRopeBlock;
  if (gy > 65535 || gx > 0x7fffffffLL) {
    set_error("eg_rope: grid too large (batch*groups=%lld)", (long long)gy);
    return 1;
  }
  EG_LAUNCH((rope_kernel<T, TT, VEC, VEC * sizeof(T) == 16>), dim3((unsigned)gx, (unsigned)gy), dim3(kRopeBlock),
                     0, st, (const T*)q, (const T*)k, (T*)qo, (T*)ko, (const TT*)cosv,
                     (const TT*)sinv, (int)hq, (int)hk, (int)tokens, (int)head_dim, gq, gk,
                     sgn);
  return check_launch("eg_rope");
}

template <typename T, typename TT>
int rope_dispatch_vec(const void* q, const void* k, void* qo, void* ko, const void* cosv,
                      const void* sinv, int64_t batch, int64_t hq, int64_t hk, int64_t tokens,
                      int64_t head_dim, float sgn, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  const int64_t half = head_dim / 2;
  const bool vec = half % V == 0 && aligned_to(q, 16) && aligned_to(k, 16) &&
                   aligned_to(qo, 16) && aligned_to(ko, 16) &&
                   aligned_to(cosv, sizeof(TT) * V) && aligned_to(sinv, sizeof(TT) * V);
  if (vec)
    return launch_rope<T, TT, V>(q, k, qo, ko, cosv, sinv, batch, hq, hk, tokens, head_dim, sgn, st);
  return launch_rope<T, TT, 1>(q, k, qo, ko, cosv, sinv, batch, hq, hk, tokens, head_dim, sgn, st);
}

}  // namespace

int rope_apply(const void* q, const void* k, void* q_out, void* k_out, const void* cos,
               const void* sin, int64_t batch, int64_t heads_q, int64_t heads_k,
               int64_t tokens, int64_t head_dim, int dtype, int table_dtype, bool inverse,
               hipStream_t st) {
  const float sgn = inverse ? -1.0f : 1.0f;
  return EG_DISPATCH_FLOAT(dtype, "eg_rope", [&] {
    using T = scalar_t;
    if (table_dtype == EG_F32)
      return rope_dispatch_vec<T, float>(q, k, q_out, k_out, cos, sin, batch, heads_q, heads_k,
                                         tokens, head_dim, sgn, st);
    return rope_dispatch_vec<T, T>(q, k, q_out, k_out, cos, sin, batch, heads_q, heads_k, tokens,
                                   head_dim, sgn, st);
  });
}

}  // namespace eg

using namespace eg;

extern "C" int eg_rope(const void* q, const void* k, void* q_out, void* k_out, const void* cos,
                       const void* sin, int64_t batch, int64_t heads_q, int64_t heads_k,
                       int64_t tokens, int64_t head_dim, int dtype, int table_dtype,
                       int inverse, void* stream) {
  clear_error();
  if (batch < 0 || heads_q < 0 || heads_k < 0 || tokens < 0 || head_dim <= 0) {
    set_error("eg_rope: bad sizes");
    return 1;
  }
  if (head_dim % 2) { set_error("eg_rope: head_dim must be even, got %lld", (long long)head_dim); return 1; }
  if (tokens > 0x3fffffff || head_dim > 0x3fffffff || heads_q > 0x3fffffff || heads_k > 0x3fffffff) {
    set_error("eg_rope: size out of range");
    return 1;
  }
  if (batch == 0 || tokens == 0 || heads_q + heads_k == 0) return 0;
  if ((heads_q > 0 && (!q || !q_out)) || (heads_k > 0 && (!k || !k_out)) || !cos || !sin) {
    set_error("eg_rope: null pointer");
    return 1;
  }
  if (table_dtype != EG_F32 && table_dtype != dtype) {
    set_error("eg_rope: table dtype must be fp32 or the tensor dtype");
    return 1;
  }
  return rope_apply(q, k, q_out, k_out, cos, sin, batch, heads_q, heads_k, tokens, head_dim,
                    dtype, table_dtype, inverse != 0, as_stream(stream));
}
