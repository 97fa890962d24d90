// Layout and elementwise steps of the Llama-3 decoder layer
// (src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:91-117) that sit
// between its products, norms and attention:
//
//   split_heads: the projection output [batch * tokens, ld] (token rows holding
//     heads x head_dim values) -> [batch, heads, tokens, head_dim], the
//     .view(batch, tokens, heads, head_dim).transpose(1, 2) of :94-96, with the
//     half-rotated RoPE of :98-99 (_apply_rope, :43-47: fp32 arithmetic, cast back)
//     applied on the way when tables are given;
//   merge_heads: the inverse layout change (attn.transpose(1, 2).reshape(...) of
//     :109), optionally with the RoPE transpose dx = dy cos + [dy2, -dy1] sin (the
//     gradient of the rotated q and k);
//   add: c = a + b (the gradient of a residual connection meeting a norm's);
//   silu_mul: act = (silu(gate.float()) * up.float()).to(dtype) (:115-116), one
//     rounding (the level-1 SwiGLU rounds silu first; the layer does not).
//
// All are HBM-bound streams. A split/merge thread owns one (token, head, chunk)
// triple, the chunk being VEC consecutive elements of the first half of the head
// and the matching VEC of the second half, so the rotation pairs stay in one
// thread and every access is a 16-byte vector when head_dim / 2 allows it.
#include "eg_common.hpp"

namespace eg {
namespace {

constexpr int kLayBlock = 256;

// MODE: 0 copy, 1 rotate (forward RoPE), 2 transpose rotation (RoPE backward).
// TO_HEADS: token rows -> head-major, else head-major -> token rows.
template <typename T, typename TT, int VEC, int MODE, bool TO_HEADS>
__global__ __launch_bounds__(kLayBlock) void heads_kernel(
    const T* __restrict__ src, T* __restrict__ dst, const TT* __restrict__ cosv,
    const TT* __restrict__ sinv, int64_t n, int tokens, int heads, int head_dim, int64_t ld) {
  const int64_t idx = (int64_t)blockIdx.x * kLayBlock + threadIdx.x;
  if (idx >= n) return;
  const int half = head_dim >> 1;
  const int cph = half / VEC;  // chunks per head
  const int64_t th = idx / cph;
  const int c = (int)(idx - th * cph) * VEC;
  const int h = (int)(th % heads);
  const int64_t bt = th / heads;  // batch * tokens + token
  const int t = (int)(bt % tokens);
  const int64_t b = bt / tokens;
  const int64_t roff = bt * ld + (int64_t)h * head_dim + c;                       // token rows
  const int64_t hoff = ((b * heads + h) * tokens + t) * (int64_t)head_dim + c;     // head-major
  const int64_t so = TO_HEADS ? roff : hoff, doff = TO_HEADS ? hoff : roff;
  float x1[VEC], x2[VEC];
  load_f32<T, VEC>(src + so, x1);
  load_f32<T, VEC>(src + so + half, x2);
  if constexpr (MODE != 0) {
    const int64_t to = (int64_t)t * head_dim + c;
    float c1[VEC], c2[VEC], s1[VEC], s2[VEC];
    load_f32<TT, VEC>(cosv + to, c1);
    load_f32<TT, VEC>(cosv + to + half, c2);
    load_f32<TT, VEC>(sinv + to, s1);
    load_f32<TT, VEC>(sinv + to + half, s2);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float a = x1[i], bb = x2[i];
      if constexpr (MODE == 1) {
        x1[i] = a * c1[i] - bb * s1[i];
        x2[i] = bb * c2[i] + a * s2[i];
      } else {
        x1[i] = a * c1[i] + bb * s2[i];
        x2[i] = bb * c2[i] - a * s1[i];
      }
    }
  }
  store_f32<T, VEC>(dst + doff, x1);
  store_f32<T, VEC>(dst + doff + half, x2);
}

// The q, k and v of one fused projection in one launch: a token row of the [rows, ld]
// buffer holds heads_q query heads, then heads_kv key heads, then heads_kv value
// heads (head_dim each, from column 0); each goes to (TO_HEADS) or comes from its own
// head-major tensor. Query and key heads take the rotation of MODE; value heads are
// copied. A thread owns one (token, head, chunk) triple as in heads_kernel.
template <typename T>
struct QkvHeads {
  T* base[3];    // head-major q, k, v: [batch, heads of each, tokens, head_dim]
  int first[4];  // first head of q, k, v in a token row, then the row's head count
};

template <typename T, typename TT, int VEC, int MODE, bool TO_HEADS>
__global__ __launch_bounds__(kLayBlock) void qkv_heads_kernel(
    const T* __restrict__ src_rows, T* __restrict__ dst_rows, QkvHeads<T> hd,
    const TT* __restrict__ cosv, const TT* __restrict__ sinv, int64_t n, int tokens,
    int head_dim, int64_t ld) {
  const int64_t idx = (int64_t)blockIdx.x * kLayBlock + threadIdx.x;
  if (idx >= n) return;
  const int heads = hd.first[3];
  const int half = head_dim >> 1;
  const int cph = half / VEC;  // chunks per head
  const int64_t th = idx / cph;
  const int c = (int)(idx - th * cph) * VEC;
  const int g = (int)(th % heads);  // head within the token row
  const int64_t bt = th / heads;    // batch * tokens + token
  const int t = (int)(bt % tokens);
  const int64_t b = bt / tokens;
  const int which = g < hd.first[1] ? 0 : (g < hd.first[2] ? 1 : 2);
  const int h = g - hd.first[which];
  const int nh = hd.first[which + 1] - hd.first[which];
  T* hb = hd.base[which];
  const int64_t roff = bt * ld + (int64_t)g * head_dim + c;
  const int64_t hoff = ((b * nh + h) * tokens + t) * (int64_t)head_dim + c;
  const T* src = TO_HEADS ? src_rows + roff : hb + hoff;
  T* dst = TO_HEADS ? hb + hoff : dst_rows + roff;
  float x1[VEC], x2[VEC];
  load_f32<T, VEC>(src, x1);
  load_f32<T, VEC>(src + half, x2);
  if (MODE != 0 && which < 2) {
    const int64_t to = (int64_t)t * head_dim + c;
    float c1[VEC], c2[VEC], s1[VEC], s2[VEC];
    load_f32<TT, VEC>(cosv + to, c1);
    load_f32<TT, VEC>(cosv + to + half, c2);
    load_f32<TT, VEC>(sinv + to, s1);
    load_f32<TT, VEC>(sinv + to + half, s2);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float a = x1[i], bb = x2[i];
      if constexpr (MODE == 1) {
        x1[i] = a * c1[i] - bb * s1[i];
        x2[i] = bb * c2[i] + a * s2[i];
      } else {
        x1[i] = a * c1[i] + bb * s2[i];
        x2[i] = bb * c2[i] - a * s1[i];
      }
    }
  }
  store_f32<T, VEC>(dst, x1);
  store_f32<T, VEC>(dst + half, x2);
}

template <typename T, int VEC>
__global__ __launch_bounds__(kLayBlock) void add_kernel(const T* __restrict__ a,
                                                        const T* __restrict__ b,
                                                        T* __restrict__ c, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * kLayBlock + threadIdx.x) * VEC;
  if (i >= n) return;
  float x[VEC], y[VEC];
  load_f32<T, VEC>(a + i, x);
  load_f32<T, VEC>(b + i, y);
#pragma unroll
  for (int e = 0; e < VEC; ++e) x[e] += y[e];
  store_f32<T, VEC>(c + i, x);
}

template <typename T, int VEC>
__global__ __launch_bounds__(kLayBlock) void silu_mul_kernel(const T* __restrict__ g,
                                                             const T* __restrict__ u,
                                                             T* __restrict__ out, int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * kLayBlock + threadIdx.x) * VEC;
  if (i >= n) return;
  float x[VEC], y[VEC];
  load_f32<T, VEC>(g + i, x);
  load_f32<T, VEC>(u + i, y);
#pragma unroll
  for (int e = 0; e < VEC; ++e) x[e] = x[e] / (1.0f + expf(-x[e])) * y[e];
  store_f32<T, VEC>(out + i, x);
}

template <typename F>
int layer_dispatch(int dtype, const char* what, F&& f) {
  switch (dtype) {
    case EG_F32: return f(float{});
    case EG_F16: return f(f16_t{});
    case EG_BF16: return f(bf16_t{});
    default: set_error("%s: unsupported dtype %d", what, dtype); return 1;
  }
}

int heads_launch(const void* src, void* dst, const void* cosv, const void* sinv, int64_t batch,
                 int64_t tokens, int64_t heads, int64_t head_dim, int64_t ld, int rope,
                 int table_dtype, int dtype, bool to_heads, void* stream, const char* name) {
  clear_error();
  if (batch < 0 || tokens < 0 || heads < 0 || head_dim < 0) {
    set_error("%s: negative size", name);
    return 1;
  }
  if (head_dim % 2 || ld < heads * head_dim) {
    set_error("%s: head_dim must be even and ld >= heads * head_dim", name);
    return 1;
  }
  if (rope < 0 || rope > 2 || (rope && (!cosv || !sinv))) {
    set_error("%s: rope must be 0 (none), 1 (rotate) or 2 (transpose) with both tables", name);
    return 1;
  }
  if (rope && table_dtype != EG_F32 && table_dtype != dtype) {
    set_error("%s: tables must be fp32 or the tensors' dtype", name);
    return 1;
  }
  const int64_t rows = batch * tokens * heads;
  if (rows == 0 || head_dim == 0) return 0;
  if (!src || !dst) {
    set_error("%s: null pointer", name);
    return 1;
  }
  if (tokens > 0x7fffffff || heads > 0x7fffffff || head_dim > 0x7fffffff) {
    set_error("%s: size out of range", name);
    return 1;
  }
  hipStream_t st = as_stream(stream);
  return layer_dispatch(dtype, name, [&](auto tag) {
    using T = decltype(tag);
    constexpr int V = 16 / sizeof(T);
    const bool vec = (head_dim / 2) % V == 0 && ld % V == 0 && aligned16(src) && aligned16(dst) &&
                     (!rope || (aligned16(cosv) && aligned16(sinv)));
    auto go = [&](auto vc, auto tt) {
      constexpr int VC = decltype(vc)::value;
      using TT = decltype(tt);
      const int64_t n = rows * (head_dim / 2 / VC);
      const unsigned grid = (unsigned)((n + kLayBlock - 1) / kLayBlock);
      auto launch = [&](auto mode, auto dir) {
        EG_LAUNCH((heads_kernel<T, TT, VC, decltype(mode)::value, decltype(dir)::value>),
                  dim3(grid), dim3(kLayBlock), 0, st, (const T*)src, (T*)dst, (const TT*)cosv,
                  (const TT*)sinv, n, (int)tokens, (int)heads, (int)head_dim, ld);
      };
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      if (to_heads) {
        if (rope == 0) launch(I0{}, std::true_type{});
        else if (rope == 1) launch(I1{}, std::true_type{});
        else launch(I2{}, std::true_type{});
      } else {
        if (rope == 0) launch(I0{}, std::false_type{});
        else if (rope == 1) launch(I1{}, std::false_type{});
        else launch(I2{}, std::false_type{});
      }
      return check_launch(name);
    };
    // the fp32 tables are read with VEC-wide loads too: a 16-byte vector holds 4
    auto pick_tables = [&](auto vc) {
      if (rope && table_dtype == EG_F32 && !std::is_same<T, float>::value)
        return go(vc, float{});
      return go(vc, T{});
    };
    // 16-bit tensors with fp32 tables read 8 table values (32 bytes) per chunk half
    if (vec) return pick_tables(std::integral_constant<int, V>{});
    return pick_tables(std::integral_constant<int, 1>{});
  });
}

int qkv_heads_launch(const void* rows_src, void* rows_dst, const void* q, const void* k,
                     const void* v, const void* cosv, const void* sinv, int64_t batch,
                     int64_t tokens, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
                     int64_t ld, int rope, int table_dtype, int dtype, bool to_heads,
                     void* stream, const char* name) {
  clear_error();
  if (batch < 0 || tokens < 0 || heads_q < 0 || heads_kv < 0 || head_dim < 0) {
    set_error("%s: negative size", name);
    return 1;
  }
  const int64_t heads = heads_q + 2 * heads_kv;
  if (head_dim % 2 || ld < heads * head_dim) {
    set_error("%s: head_dim must be even and ld >= (heads_q + 2 heads_kv) * head_dim", name);
    return 1;
  }
  if (rope < 0 || rope > 2 || (rope && (!cosv || !sinv))) {
    set_error("%s: rope must be 0 (none), 1 (rotate) or 2 (transpose) with both tables", name);
    return 1;
  }
  if (rope && table_dtype != EG_F32 && table_dtype != dtype) {
    set_error("%s: tables must be fp32 or the tensors' dtype", name);
    return 1;
  }
  const int64_t rows = batch * tokens * heads;
  if (rows == 0 || head_dim == 0) return 0;
  const void* rows_ptr = to_heads ? rows_src : rows_dst;
  if (!rows_ptr || (heads_q && !q) || (heads_kv && (!k || !v))) {
    set_error("%s: null pointer", name);
    return 1;
  }
  if (tokens > 0x7fffffff || heads > 0x7fffffff || head_dim > 0x7fffffff) {
    set_error("%s: size out of range", name);
    return 1;
  }
  hipStream_t st = as_stream(stream);
  return layer_dispatch(dtype, name, [&](auto tag) {
    using T = decltype(tag);
    constexpr int V = 16 / sizeof(T);
    QkvHeads<T> hd;
    hd.base[0] = (T*)q;
    hd.base[1] = (T*)k;
    hd.base[2] = (T*)v;
    hd.first[0] = 0;
    hd.first[1] = (int)heads_q;
    hd.first[2] = (int)(heads_q + heads_kv);
    hd.first[3] = (int)heads;
    const bool vec = (head_dim / 2) % V == 0 && ld % V == 0 && aligned16(rows_ptr) &&
                     (!heads_q || aligned16(q)) && (!heads_kv || (aligned16(k) && aligned16(v))) &&
                     (!rope || (aligned16(cosv) && aligned16(sinv)));
    auto go = [&](auto vc, auto tt) {
      constexpr int VC = decltype(vc)::value;
      using TT = decltype(tt);
      const int64_t n = rows * (head_dim / 2 / VC);
      const unsigned grid = (unsigned)((n + kLayBlock - 1) / kLayBlock);
      auto launch = [&](auto mode, auto dir) {
        EG_LAUNCH((qkv_heads_kernel<T, TT, VC, decltype(mode)::value, decltype(dir)::value>),
                  dim3(grid), dim3(kLayBlock), 0, st, (const T*)rows_src, (T*)rows_dst, hd,
                  (const TT*)cosv, (const TT*)sinv, n, (int)tokens, (int)head_dim, ld);
      };
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      if (to_heads) {
        if (rope == 0) launch(I0{}, std::true_type{});
        else if (rope == 1) launch(I1{}, std::true_type{});
        else launch(I2{}, std::true_type{});
      } else {
        if (rope == 0) launch(I0{}, std::false_type{});
        else if (rope == 1) launch(I1{}, std::false_type{});
        else launch(I2{}, std::false_type{});
      }
      return check_launch(name);
    };
    auto pick_tables = [&](auto vc) {
      if (rope && table_dtype == EG_F32 && !std::is_same<T, float>::value)
        return go(vc, float{});
      return go(vc, T{});
    };
    if (vec) return pick_tables(std::integral_constant<int, V>{});
    return pick_tables(std::integral_constant<int, 1>{});
  });
}

}  // namespace
}  // namespace eg

using namespace eg;

extern "C" int eg_split_qkv_heads(const void* src, void* q, void* k, void* v, const void* cos,
                                  const void* sin, int64_t batch, int64_t tokens,
                                  int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t ld,
                                  int rope, int table_dtype, int dtype, void* stream) {
  return qkv_heads_launch(src, nullptr, q, k, v, cos, sin, batch, tokens, heads_q, heads_kv,
                          head_dim, ld, rope, table_dtype, dtype, true, stream,
                          "eg_split_qkv_heads");
}

extern "C" int eg_merge_qkv_heads(const void* q, const void* k, const void* v, void* dst,
                                  const void* cos, const void* sin, int64_t batch, int64_t tokens,
                                  int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t ld,
                                  int rope, int table_dtype, int dtype, void* stream) {
  return qkv_heads_launch(nullptr, dst, q, k, v, cos, sin, batch, tokens, heads_q, heads_kv,
                          head_dim, ld, rope, table_dtype, dtype, false, stream,
                          "eg_merge_qkv_heads");
}

extern "C" int eg_split_heads(const void* src, void* dst, const void* cos, const void* sin,
                              int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim,
                              int64_t ld, int rope, int table_dtype, int dtype, void* stream) {
  return heads_launch(src, dst, cos, sin, batch, tokens, heads, head_dim, ld, rope, table_dtype,
                      dtype, true, stream, "eg_split_heads");
}

extern "C" int eg_merge_heads(const void* src, void* dst, const void* cos, const void* sin,
                              int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim,
                              int64_t ld, int rope, int table_dtype, int dtype, void* stream) {
  return heads_launch(src, dst, cos, sin, batch, tokens, heads, head_dim, ld, rope, table_dtype,
                      dtype, false, stream, "eg_merge_heads");
}

extern "C" int eg_add(const void* a, const void* b, void* c, int64_t n, int dtype,
                      void* stream) {
  clear_error();
  if (n < 0) {
    set_error("eg_add: negative size");
    return 1;
  }
  if (n == 0) return 0;
  if (!a || !b || !c) {
    set_error("eg_add: null pointer");
    return 1;
  }
  hipStream_t st = as_stream(stream);
  return layer_dispatch(dtype, "eg_add", [&](auto tag) {
    using T = decltype(tag);
    constexpr int V = 16 / sizeof(T);
    if (n % V == 0 && aligned16(a) && aligned16(b) && aligned16(c)) {
      const int64_t nb = (n / V + kLayBlock - 1) / kLayBlock;
      EG_LAUNCH((add_kernel<T, V>), dim3((unsigned)nb), dim3(kLayBlock), 0, st, (const T*)a,
                (const T*)b, (T*)c, n);
    } else {
      EG_LAUNCH((add_kernel<T, 1>), dim3((unsigned)((n + kLayBlock - 1) / kLayBlock)),
                dim3(kLayBlock), 0, st, (const T*)a, (const T*)b, (T*)c, n);
    }
    return check_launch("eg_add");
  });
}

extern "C" int eg_silu_mul(const void* gate, const void* up, void* out, int64_t n, int dtype,
                           void* stream) {
  clear_error();
  if (n < 0) {
    set_error("eg_silu_mul: negative size");
    return 1;
  }
  if (n == 0) return 0;
  if (!gate || !up || !out) {
    set_error("eg_silu_mul: null pointer");
    return 1;
  }
  hipStream_t st = as_stream(stream);
  return layer_dispatch(dtype, "eg_silu_mul", [&](auto tag) {
    using T = decltype(tag);
    constexpr int V = 16 / sizeof(T);
    if (n % V == 0 && aligned16(gate) && aligned16(up) && aligned16(out)) {
      const int64_t nb = (n / V + kLayBlock - 1) / kLayBlock;
      EG_LAUNCH((silu_mul_kernel<T, V>), dim3((unsigned)nb), dim3(kLayBlock), 0, st,
                (const T*)gate, (const T*)up, (T*)out, n);
    } else {
      EG_LAUNCH((silu_mul_kernel<T, 1>), dim3((unsigned)((n + kLayBlock - 1) / kLayBlock)),
                dim3(kLayBlock), 0, st, (const T*)gate, (const T*)up, (T*)out, n);
    }
    return check_launch("eg_silu_mul");
  });
}
