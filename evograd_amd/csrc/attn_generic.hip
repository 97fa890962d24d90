// Causal (grouped-query) attention for the shapes the MFMA kernels do not take:
// fp32 tensors, and head sizes other than 64 and 128 in any dtype.
//
// Same contract as attention.hip (F.scaled_dot_product_attention(q, k, v,
// is_causal=True) as called by src/evograd/ops/level3/llama3_decoder_layer/
// forward_ref.py:107, with the kv head of query head h being h / (H / Hkv), the
// repeat_interleave of :101-105): o = softmax(q k^T * scale + causal mask) v, lse =
// logsumexp of the scaled, masked scores (natural log, fp32), and the backward
// dq, dk, dv with P recomputed from lse and delta = rowsum(do * o).
//
// The reference's decoder layer gates its algebra at fp32 with head_dim 32 and 16
// (src/evograd/ops/level3/llama3_decoder_layer/__init__.py:55-65); these kernels
// serve that gate and any other shape outside the MFMA path. They are plain fp32
// arithmetic on 64-thread workgroups (one wave), one query row (forward, dQ) or one
// key row (dK/dV) per lane, with the other operand's 64-row tiles staged in LDS in
// fp32: every lane reads the same LDS row at a time (a broadcast), and each lane
// keeps its row and accumulators in registers. DM (16, 32, 64 or 128) is the
// largest head size an instantiation takes; the runtime head size D <= DM.
// No atomics: dQ and dK/dV are separate kernels, each a fixed-order sum.
#include "eg_common.hpp"

namespace eg {
namespace {

constexpr int kGenRows = 64;
constexpr float kGenLog2e = 1.4426950408889634f;
constexpr float kGenLn2 = 0.6931471805599453f;

// Loads rows r0 .. r0 + 63 of a [S, D] slice into LDS as fp32 (rows past S as zero).
template <typename T, int DM>
__device__ __forceinline__ void stage_rows(float* __restrict__ lds, const T* __restrict__ src,
                                           int r0, int S, int D) {
  for (int e = threadIdx.x; e < kGenRows * D; e += kGenRows) {
    const int r = e / D, d = e - r * D;
    lds[r * DM + d] = (r0 + r < S) ? to_f32(src[(int64_t)(r0 + r) * D + d]) : 0.f;
  }
}

// Row x of position t rotated by the tables (rotate-half convention): forward
// y = x cos + [-x2, x1] sin; transpose dx = dy cos + [dy2, -dy1] sin.
template <int DM>
__device__ __forceinline__ void rotate_row(float (&x)[DM], const float* __restrict__ rc,
                                           const float* __restrict__ rs, int t, int D,
                                           bool transpose) {
  const int half = D / 2;
  float y[DM];
#pragma unroll
  for (int d = 0; d < DM; ++d) {
    if (d >= D) { y[d] = 0.f; continue; }
    const float c = rc[(int64_t)t * D + d], s = rs[(int64_t)t * D + d];
    float other = 0.f;
    // the partner element of d in the other half (d +/- half), picked without a
    // dynamic register index
#pragma unroll
    for (int e = 0; e < DM; ++e)
      if (e < D && (e == d + half || e == d - half)) other = x[e];
    const float rot = (d < half) ? (transpose ? other : -other) : (transpose ? -other : other);
    if (!transpose) {
      y[d] = x[d] * c + rot * s;
    } else {
      // transpose: dx_d = dy_d c_d + (d < half ? dy_{d+half} s_{d+half} : -dy_{d-half} s_{d-half})
      const int p = d < half ? d + half : d - half;
      const float sp = rs[(int64_t)t * D + p];
      y[d] = x[d] * c + rot * sp;
    }
  }
#pragma unroll
  for (int d = 0; d < DM; ++d) x[d] = y[d];
}

// Forward: workgroup (query block qb, slice bh); lane = one query row.
template <typename T, int DM, bool ROPE>
__global__ __launch_bounds__(kGenRows) void attn_gen_fwd_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, T* __restrict__ o,
    float* __restrict__ lse, int S, int D, int H, int group, float scale_log2,
    const float* __restrict__ rc, const float* __restrict__ rs) {
  __shared__ float Ks[kGenRows * DM], Vs[kGenRows * DM];
  const int bh = blockIdx.y;
  const int64_t bhk = (int64_t)(bh / H) * (H / group) + (bh % H) / group;
  const int i0 = blockIdx.x * kGenRows, i = i0 + threadIdx.x;
  const bool live = i < S;
  const T* qs = q + (int64_t)bh * S * D;
  const T* ks = k + bhk * S * D;
  const T* vs = v + bhk * S * D;
  float qv[DM], acc[DM];
#pragma unroll
  for (int d = 0; d < DM; ++d) {
    qv[d] = (live && d < D) ? to_f32(qs[(int64_t)i * D + d]) : 0.f;
    acc[d] = 0.f;
  }
  if constexpr (ROPE) {
    if (live) rotate_row<DM>(qv, rc, rs, i, D, false);
  }
#pragma unroll
  for (int d = 0; d < DM; ++d) qv[d] *= scale_log2;
  float m = -INFINITY, l = 0.f;
  for (int j0 = 0; j0 <= i0 && j0 < S; j0 += kGenRows) {
    __syncthreads();
    stage_rows<T, DM>(Ks, ks, j0, S, D);
    stage_rows<T, DM>(Vs, vs, j0, S, D);
    __syncthreads();
    const int jn = min(kGenRows, S - j0);
    for (int jj = 0; jj < jn; ++jj) {
      if (!live || j0 + jj > i) continue;
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < DM; ++d)
        if (d < D) s = __builtin_fmaf(qv[d], Ks[jj * DM + d], s);
      const float mn = fmaxf(m, s);
      const float corr = __builtin_amdgcn_exp2f(m - mn);
      const float p = __builtin_amdgcn_exp2f(s - mn);
      l = l * corr + p;
#pragma unroll
      for (int d = 0; d < DM; ++d)
        if (d < D) acc[d] = __builtin_fmaf(p, Vs[jj * DM + d], acc[d] * corr);
      m = mn;
    }
  }
  if (!live) return;
  const float inv = 1.f / l;
  T* os = o + (int64_t)bh * S * D + (int64_t)i * D;
#pragma unroll
  for (int d = 0; d < DM; ++d)
    if (d < D) os[d] = from_f32<T>(acc[d] * inv);
  lse[(int64_t)bh * S + i] = (m + __log2f(l)) * kGenLn2;
}

// dQ (and delta = rowsum(do * o) for the dK/dV kernel): lane = one query row.
template <typename T, int DM, bool ROPE>
__global__ __launch_bounds__(kGenRows) void attn_gen_dq_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ dout, const T* __restrict__ o, const float* __restrict__ lse,
    float* __restrict__ delta, T* __restrict__ dq, int S, int D, int H, int group, float scale,
    const float* __restrict__ rc, const float* __restrict__ rs) {
  __shared__ float Ks[kGenRows * DM], Vs[kGenRows * DM];
  const int bh = blockIdx.y;
  const int64_t bhk = (int64_t)(bh / H) * (H / group) + (bh % H) / group;
  const int i0 = blockIdx.x * kGenRows, i = i0 + threadIdx.x;
  const bool live = i < S;
  const int64_t row = (int64_t)bh * S * D + (int64_t)i * D;
  const T* ks = k + bhk * S * D;
  const T* vs = v + bhk * S * D;
  const float sl2 = scale * kGenLog2e;
  float qv[DM], dov[DM], acc[DM];
  float dl = 0.f;
#pragma unroll
  for (int d = 0; d < DM; ++d) {
    qv[d] = (live && d < D) ? to_f32(q[row + d]) * sl2 : 0.f;
    dov[d] = (live && d < D) ? to_f32(dout[row + d]) : 0.f;
    const float ov = (live && d < D) ? to_f32(o[row + d]) : 0.f;
    dl = __builtin_fmaf(dov[d], ov, dl);
    acc[d] = 0.f;
  }
  const float l2 = live ? lse[(int64_t)bh * S + i] * kGenLog2e : 0.f;
  if (live) delta[(int64_t)bh * S + i] = dl;
  for (int j0 = 0; j0 <= i0 && j0 < S; j0 += kGenRows) {
    __syncthreads();
    stage_rows<T, DM>(Ks, ks, j0, S, D);
    stage_rows<T, DM>(Vs, vs, j0, S, D);
    __syncthreads();
    const int jn = min(kGenRows, S - j0);
    for (int jj = 0; jj < jn; ++jj) {
      if (!live || j0 + jj > i) continue;
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int d = 0; d < DM; ++d)
        if (d < D) {
          s = __builtin_fmaf(qv[d], Ks[jj * DM + d], s);
          dp = __builtin_fmaf(dov[d], Vs[jj * DM + d], dp);
        }
      const float ds = __builtin_amdgcn_exp2f(s - l2) * (dp - dl);
#pragma unroll
      for (int d = 0; d < DM; ++d)
        if (d < D) acc[d] = __builtin_fmaf(ds, Ks[jj * DM + d], acc[d]);
    }
  }
  if (!live) return;
#pragma unroll
  for (int d = 0; d < DM; ++d) acc[d] *= scale;
  if constexpr (ROPE) rotate_row<DM>(acc, rc, rs, i, D, true);
#pragma unroll
  for (int d = 0; d < DM; ++d)
    if (d < D) dq[row + d] = from_f32<T>(acc[d]);
}

// dK, dV: workgroup (key block kb, kv slice); lane = one key row; the query heads
// of the group are walked in order, each over the query blocks at or after kb.
template <typename T, int DM, bool ROPE>
__global__ __launch_bounds__(kGenRows) void attn_gen_dkdv_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ dout, const float* __restrict__ lse, const float* __restrict__ delta,
    T* __restrict__ dk, T* __restrict__ dv, int S, int D, int Hkv, int group, float scale,
    const float* __restrict__ rc, const float* __restrict__ rs) {
  __shared__ float Qs[kGenRows * DM], Ds[kGenRows * DM];
  __shared__ float Ls[kGenRows], Dl[kGenRows];
  const int bhk = blockIdx.y;
  const int b = bhk / Hkv, hk = bhk % Hkv;
  const int H = Hkv * group;
  const int j0 = blockIdx.x * kGenRows, j = j0 + threadIdx.x;
  const bool live = j < S;
  const int64_t row = (int64_t)bhk * S * D + (int64_t)j * D;
  const float sl2 = scale * kGenLog2e;
  float kv[DM], vv[DM], adk[DM], adv[DM];
#pragma unroll
  for (int d = 0; d < DM; ++d) {
    kv[d] = (live && d < D) ? to_f32(k[row + d]) * sl2 : 0.f;
    vv[d] = (live && d < D) ? to_f32(v[row + d]) : 0.f;
    adk[d] = 0.f;
    adv[d] = 0.f;
  }
  for (int g = 0; g < group; ++g) {
    const int64_t bh = (int64_t)b * H + (int64_t)hk * group + g;
    const T* qs = q + bh * S * D;
    const T* dos = dout + bh * S * D;
    for (int i0 = j0; i0 < S; i0 += kGenRows) {
      __syncthreads();
      stage_rows<T, DM>(Qs, qs, i0, S, D);
      stage_rows<T, DM>(Ds, dos, i0, S, D);
      {
        const int r = i0 + threadIdx.x;
        Ls[threadIdx.x] = r < S ? lse[bh * S + r] * kGenLog2e : 0.f;
        Dl[threadIdx.x] = r < S ? delta[bh * S + r] : 0.f;
      }
      __syncthreads();
      const int in = min(kGenRows, S - i0);
      for (int ii = 0; ii < in; ++ii) {
        if (!live || i0 + ii < j) continue;
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int d = 0; d < DM; ++d)
          if (d < D) {
            s = __builtin_fmaf(kv[d], Qs[ii * DM + d], s);
            dp = __builtin_fmaf(vv[d], Ds[ii * DM + d], dp);
          }
        const float p = __builtin_amdgcn_exp2f(s - Ls[ii]);
        const float ds = p * (dp - Dl[ii]);
#pragma unroll
        for (int d = 0; d < DM; ++d)
          if (d < D) {
            adv[d] = __builtin_fmaf(p, Ds[ii * DM + d], adv[d]);
            adk[d] = __builtin_fmaf(ds, Qs[ii * DM + d], adk[d]);
          }
      }
    }
  }
  if (!live) return;
#pragma unroll
  for (int d = 0; d < DM; ++d) adk[d] *= scale;
  if constexpr (ROPE) rotate_row<DM>(adk, rc, rs, j, D, true);
#pragma unroll
  for (int d = 0; d < DM; ++d)
    if (d < D) {
      dk[row + d] = from_f32<T>(adk[d]);
      dv[row + d] = from_f32<T>(adv[d]);
    }
}

template <typename F>
int gen_dispatch(int dtype, int64_t D, const char* name, F&& f) {
  auto by_dim = [&](auto tag) -> int {
    if (D <= 16) return f(tag, std::integral_constant<int, 16>{});
    if (D <= 32) return f(tag, std::integral_constant<int, 32>{});
    if (D <= 64) return f(tag, std::integral_constant<int, 64>{});
    return f(tag, std::integral_constant<int, 128>{});
  };
  switch (dtype) {
    case EG_F32: return by_dim(float{});
    case EG_F16: return by_dim(f16_t{});
    case EG_BF16: return by_dim(bf16_t{});
    default: set_error("%s: unsupported dtype %d", name, dtype); return 1;
  }
}

}  // namespace

int attn_generic_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B,
                     int64_t H, int64_t Hkv, int64_t S, int64_t D, float scale, int dtype,
                     hipStream_t st, const float* rc, const float* rs) {
  const dim3 grid((unsigned)((S + kGenRows - 1) / kGenRows), (unsigned)(B * H));
  const int group = (int)(H / Hkv);
  return gen_dispatch(dtype, D, "eg_attn_fwd", [&](auto tag, auto dm) {
    using T = decltype(tag);
    constexpr int DM = decltype(dm)::value;
    if (rc)
      EG_LAUNCH((attn_gen_fwd_kernel<T, DM, true>), grid, dim3(kGenRows), 0, st, (const T*)q,
                (const T*)k, (const T*)v, (T*)o, lse, (int)S, (int)D, (int)H, group,
                scale * kGenLog2e, rc, rs);
    else
      EG_LAUNCH((attn_gen_fwd_kernel<T, DM, false>), grid, dim3(kGenRows), 0, st, (const T*)q,
                (const T*)k, (const T*)v, (T*)o, lse, (int)S, (int)D, (int)H, group,
                scale * kGenLog2e, rc, rs);
    return check_launch("eg_attn_fwd(generic)");
  });
}

int attn_generic_bwd(const void* dout, const void* q, const void* k, const void* v,
                     const void* o, const float* lse, void* dq, void* dk, void* dv, float* delta,
                     int64_t B, int64_t H, int64_t Hkv, int64_t S, int64_t D, float scale,
                     int dtype, hipStream_t st, const float* rc, const float* rs) {
  const unsigned nb = (unsigned)((S + kGenRows - 1) / kGenRows);
  const int group = (int)(H / Hkv);
  return gen_dispatch(dtype, D, "eg_attn_bwd", [&](auto tag, auto dm) {
    using T = decltype(tag);
    constexpr int DM = decltype(dm)::value;
    auto go = [&](auto rope) {
      constexpr bool R = decltype(rope)::value;
      EG_LAUNCH((attn_gen_dq_kernel<T, DM, R>), dim3(nb, (unsigned)(B * H)), dim3(kGenRows), 0, st,
                (const T*)q, (const T*)k, (const T*)v, (const T*)dout, (const T*)o, lse, delta,
                (T*)dq, (int)S, (int)D, (int)H, group, scale, rc, rs);
      if (int e = check_launch("eg_attn_bwd(generic dq)")) return e;
      EG_LAUNCH((attn_gen_dkdv_kernel<T, DM, R>), dim3(nb, (unsigned)(B * Hkv)), dim3(kGenRows), 0,
                st, (const T*)q, (const T*)k, (const T*)v, (const T*)dout, lse, delta, (T*)dk,
                (T*)dv, (int)S, (int)D, (int)Hkv, group, scale, rc, rs);
      return check_launch("eg_attn_bwd(generic dkdv)");
    };
    return rc ? go(std::true_type{}) : go(std::false_type{});
  });
}

}  // namespace eg
