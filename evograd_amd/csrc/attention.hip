// Causal scaled-dot-product attention forward/backward for gfx950 (bf16/fp16
// operands, fp32 accumulation on MFMA).
//
// Semantics: F.scaled_dot_product_attention(q, k, v, is_causal=True) as used by
// src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:107:
//   o = softmax(q k^T * scale + causal mask) v,   lse = logsumexp(q k^T * scale + mask)
// Backward recomputes P = exp(q k^T * scale - lse) and, with delta = rowsum(do * o):
//   dv = P^T do,  dS = P * (do v^T - delta),  dq = scale * dS k,  dk = scale * dS^T q.
//
// Layout: q, k, v, o, do, dq, dk, dv are [B, H, S, D] row-major (D contiguous);
// lse and delta are fp32 [B, H, S].
//
// MFMA: v_mfma_f32_32x32x16_{bf16,f16}. Lane l of a wave holds, for an M x K
// operand A, row l%32 and k = 8*(l/32) .. +7 (16 contiguous bytes when k runs
// along memory); for B (K x N), column l%32 and the same k; the 32 x 32 fp32
// result C gives lane l column l%32 and, in register r, row (r/4)*8 + (l/32)*4 + r%4.
// Every product is arranged so that its result feeds the next one without a
// shuffle: a result C (M x N) is the B operand of X * C, with the k index of that
// product permuted to C's register order (rows 8j + 4*(l/32) + i). The matching A
// operand is read from an LDS copy stored transposed with that permutation applied
// to each 16-wide group ([0-3, 8-11, 4-7, 12-15]), so each operand fetch is one
// 16-byte LDS read. Transposed tiles are 64 wide; their eight 16-byte groups are
// XOR-swizzled by (row / 8) % 8 so that both the transposing 8-byte writes and
// the 16-byte operand reads spread over the LDS banks.
//
// Kernels (all deterministic, no atomics):
//   attn_fwd:    one workgroup = 128 query rows of one (b, h) (4 waves x 32 rows);
//                loops over 64-key tiles up to the diagonal; online softmax in the
//                log2 domain with the running max refreshed only when it grows by
//                more than 2^8 (exact: the reference point cancels in o = sum/l);
//                S^T = K Q^T then O^T += V^T P^T.
//   attn_delta:  delta = rowsum(do * o).
//   attn_dkdv:   one workgroup = 128 keys (4 waves x 32 keys); loops over 64-row
//                query tiles from the diagonal down; S = Q K^T, dP = dO V^T,
//                dV^T += dO^T P, dK^T += Q^T dS.
//   attn_dq:     one workgroup = 128 query rows; loops over 64-key tiles;
//                S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T.
#include "eg_common.hpp"

#include <initializer_list>

namespace eg {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T> struct MM;
template <> struct MM<bf16_t> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack2_bf16(lo, hi); }
};
template <> struct MM<f16_t> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack2_f16(lo, hi); }
};

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleThreshold = 8.0f;  // log2 units: refresh the max past 2^8 growth

template <typename V>
__device__ __forceinline__ V ld16(const uint16_t* p) {
  return *reinterpret_cast<const V*>(p);
}

// Eight fp32 values (registers off..off+7 of a result tile) rounded and packed
// as one MFMA operand.
template <typename T>
__device__ __forceinline__ typename MM<T>::v8 pack8(const f32x16& c, int off) {
  uint4 u;
  u.x = MM<T>::pack2(c[off + 0], c[off + 1]);
  u.y = MM<T>::pack2(c[off + 2], c[off + 3]);
  u.z = MM<T>::pack2(c[off + 4], c[off + 5]);
  u.w = MM<T>::pack2(c[off + 6], c[off + 7]);
  typename MM<T>::v8 r;
  __builtin_memcpy(&r, &u, 16);
  return r;
}

// Four fp32 values scaled by `f`, packed as 8 bytes.
template <typename T>
__device__ __forceinline__ uint2 pack4(const f32x16& c, int off, float f) {
  uint2 u;
  u.x = MM<T>::pack2(c[off + 0] * f, c[off + 1] * f);
  u.y = MM<T>::pack2(c[off + 2] * f, c[off + 3] * f);
  return u;
}

// Transposed 64-wide tile: element offset of (row, position `pos` of the
// permuted 64 columns). The 4-element chunks of each 16-group are stored in the
// order 0, 2, 1, 3, and the 16-byte groups are XOR-swizzled by row.
__device__ __forceinline__ int tperm(int i) {
  const int c = (i >> 2) & 3;
  return (i & ~15) | ((((c & 1) << 1) | (c >> 1)) << 2) | (i & 3);
}
__device__ __forceinline__ int toff(int row, int stride, int pos) {
  return row * stride + ((((pos >> 3) ^ (row >> 3)) & 7) << 3) + (pos & 7);
}

// Element e (0..7) of a 16-byte pack of 16-bit values.
__device__ __forceinline__ uint32_t half_of(const uint4& u, int e) {
  const uint32_t word = (e >> 1) == 0 ? u.x : (e >> 1) == 1 ? u.y : (e >> 1) == 2 ? u.z : u.w;
  return (e & 1) ? (word >> 16) : (word & 0xffffu);
}

// A 64 x D tile copied from HBM as 4-row x 8-column blocks, one block per
// thread (D = 64 has 128 blocks: threads t and t + 128 carry the same block and
// write the same values). Rows at or past `nrows` read as zero; the loads are
// unconditional (clamped address + select) so no branch hides their wait.
template <int D>
struct Tile64 {
  static constexpr int CB = D / 8;
  static constexpr int COMBOS = 16 * CB;
  uint4 r[4];

  __device__ __forceinline__ int combo() const { return (int)threadIdx.x & (COMBOS - 1); }

  __device__ __forceinline__ void load(const uint16_t* __restrict__ src, int row0, int nrows) {
    const int t = combo();
    const int rb = t / CB, cb = t - (t / CB) * CB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = row0 + 4 * rb + i;
      const int rc = row < nrows ? row : nrows - 1;
      const uint4 v = *reinterpret_cast<const uint4*>(src + (int64_t)rc * D + 8 * cb);
      r[i] = row < nrows ? v : make_uint4(0, 0, 0, 0);
    }
  }

  __device__ __forceinline__ void store_rows(uint16_t* lds, int stride) const {
    const int t = combo();
    const int rb = t / CB, cb = t - (t / CB) * CB;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<uint4*>(lds + (4 * rb + i) * stride + 8 * cb) = r[i];
  }

  // Transposed: column c of the source becomes LDS row c; source row i goes to
  // permuted position tperm(i).
  __device__ __forceinline__ void store_cols(uint16_t* lds, int stride) const {
    const int t = combo();
    const int rb = t / CB, cb = t - (t / CB) * CB;
    const int pos = tperm(4 * rb);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint2 u;
      u.x = half_of(r[0], e) | (half_of(r[1], e) << 16);
      u.y = half_of(r[2], e) | (half_of(r[3], e) << 16);
      *reinterpret_cast<uint2*>(lds + toff(8 * cb + e, stride, pos)) = u;
    }
  }
};

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// ------------------------------------------------------------------ forward
template <typename T, int D>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, uint16_t* __restrict__ o, float* __restrict__ lse, int S,
    float scale_log2, int nqb) {
  using v8 = typename MM<T>::v8;
  constexpr int BM = 128, BN = 64;
  constexpr int KSTEPS = D / 16;
  constexpr int DT = D / 32;
  constexpr int KST = D + 8;   // K row stride (elements)
  constexpr int VST = BN + 8;  // V^T row stride
  __shared__ __align__(16) uint16_t Ks[BN * KST];
  __shared__ __align__(16) uint16_t Vt[D * VST];

  const int bh = blockIdx.y;
  const int qb = nqb - 1 - (int)blockIdx.x;  // longest rows first
  const int q0 = qb * BM;
  const int lane = threadIdx.x & 63, w = wave_id();
  const int l32 = lane & 31, hh = lane >> 5;
  const int64_t base = (int64_t)bh * S * D;
  const uint16_t* qp = q + base;
  const uint16_t* kp = k + base;
  const uint16_t* vp = v + base;

  const int qrow = q0 + 32 * w + l32;
  const int qrc = qrow < S ? qrow : S - 1;
  v8 qf[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    const v8 t = ld16<v8>(qp + (int64_t)qrc * D + kk * 16 + 8 * hh);
    qf[kk] = qrow < S ? t : v8{};
  }

  f32x16 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x16{};
  float m = -INFINITY, lsum = 0.f;

  const int kv_end = min(S, q0 + BM);
  const int ntiles = (kv_end + BN - 1) / BN;
  const int wave_first_row = q0 + 32 * w;

  Tile64<D> kt, vt;
  kt.load(kp, 0, S);
  vt.load(vp, 0, S);
  for (int j = 0; j < ntiles; ++j) {
    __syncthreads();
    kt.store_rows(Ks, KST);
    vt.store_cols(Vt, VST);
    __syncthreads();
    const int k0 = j * BN;
    if (j + 1 < ntiles) {
      kt.load(kp, k0 + BN, S);
      vt.load(vp, k0 + BN, S);
    }
    if (k0 > wave_first_row + 31) continue;  // every key of the tile is above this wave's rows

    f32x16 s[2];
#pragma unroll
    for (int T2 = 0; T2 < 2; ++T2) s[T2] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk)
#pragma unroll
      for (int T2 = 0; T2 < 2; ++T2)
        s[T2] = MM<T>::mma(ld16<v8>(Ks + (32 * T2 + l32) * KST + kk * 16 + 8 * hh), qf[kk], s[T2]);

    float mt = -INFINITY;
    if (k0 + BN - 1 > wave_first_row) {  // tile crosses the diagonal for this wave
#pragma unroll
      for (int T2 = 0; T2 < 2; ++T2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 32 * T2 + (r >> 2) * 8 + 4 * hh + (r & 3);
          const float x = key > qrow ? -INFINITY : s[T2][r] * scale_log2;
          s[T2][r] = x;
          mt = fmaxf(mt, x);
        }
    } else {
#pragma unroll
      for (int T2 = 0; T2 < 2; ++T2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float x = s[T2][r] * scale_log2;
          s[T2][r] = x;
          mt = fmaxf(mt, x);
        }
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    // Refresh the reference max only when some row's max grew past the
    // threshold (always on the first tile, where m is -inf).
    if (__builtin_amdgcn_ballot_w64(mt > m + kRescaleThreshold) != 0) {
      const float m_new = fmaxf(m, mt);
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);
      lsum *= alpha;
#pragma unroll
      for (int t = 0; t < DT; ++t) acc[t] *= alpha;
      m = m_new;
    }
    const float m_use = m == -INFINITY ? 0.f : m;
    float ps = 0.f;
#pragma unroll
    for (int T2 = 0; T2 < 2; ++T2)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(s[T2][r] - m_use);
        s[T2][r] = p;
        ps += p;
      }
    lsum += ps;
#pragma unroll
    for (int ms = 0; ms < BN / 16; ++ms) {
      const v8 pb = pack8<T>(s[ms >> 1], 8 * (ms & 1));
#pragma unroll
      for (int t = 0; t < DT; ++t)
        acc[t] = MM<T>::mma(ld16<v8>(Vt + toff(32 * t + l32, VST, ms * 16 + 8 * hh)), pb, acc[t]);
    }
  }

  const float ltot = lsum + __shfl_xor(lsum, 32, 64);
  if (qrow < S) {
    const float inv = 1.0f / ltot;
    uint16_t* op = o + base + (int64_t)qrow * D;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<uint2*>(op + 32 * t + 8 * g + 4 * hh) = pack4<T>(acc[t], 4 * g, inv);
    if (hh == 0) lse[(int64_t)bh * S + qrow] = (m + log2f(ltot)) * kLn2;
  }
}

// ------------------------------------------------------------ delta = do.o
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_delta_kernel(const uint16_t* __restrict__ dout,
                                                         const uint16_t* __restrict__ o,
                                                         float* __restrict__ delta,
                                                         int64_t nrows) {
  // D/8 lanes per row, 16-byte loads.
  constexpr int LPR = D / 8;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / LPR;
  const int sub = (int)(gid % LPR);
  float s = 0.f;
  if (row < nrows) {
    float a[8], b[8];
    load_f32<T, 8>(reinterpret_cast<const T*>(dout) + row * D + sub * 8, a);
    load_f32<T, 8>(reinterpret_cast<const T*>(o) + row * D + sub * 8, b);
#pragma unroll
    for (int i = 0; i < 8; ++i) s += a[i] * b[i];
  }
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if (row < nrows && sub == 0) delta[row] = s;
}

// ------------------------------------------------------------ dK, dV
template <typename T, int D>
__global__ __launch_bounds__(256, 1) void attn_dkdv_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, uint16_t* __restrict__ dk,
    uint16_t* __restrict__ dv, int S, float scale, float scale_log2, int nkb) {
  using v8 = typename MM<T>::v8;
  constexpr int BK = 128, BQ = 64;
  constexpr int KSTEPS = D / 16;
  constexpr int DT = D / 32;
  constexpr int RST = D + 8;   // row-major tile stride
  constexpr int TST = BQ + 8;  // transposed tile stride
  __shared__ __align__(16) uint16_t Qs[BQ * RST];
  __shared__ __align__(16) uint16_t Ds[BQ * RST];
  __shared__ __align__(16) uint16_t Qt[D * TST];
  __shared__ __align__(16) uint16_t Dt[D * TST];
  __shared__ __align__(16) float Ls[BQ];
  __shared__ __align__(16) float Es[BQ];

  const int bh = blockIdx.y;
  const int kb = nkb - 1 - (int)blockIdx.x;
  const int k0 = kb * BK;
  const int lane = threadIdx.x & 63, w = wave_id();
  const int l32 = lane & 31, hh = lane >> 5;
  const int64_t base = (int64_t)bh * S * D;
  const float* lsep = lse + (int64_t)bh * S;
  const float* delp = delta + (int64_t)bh * S;

  const int key = k0 + 32 * w + l32;
  const int krc = key < S ? key : S - 1;
  v8 kf[KSTEPS], vf[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    const v8 a = ld16<v8>(k + base + (int64_t)krc * D + kk * 16 + 8 * hh);
    const v8 b = ld16<v8>(v + base + (int64_t)krc * D + kk * 16 + 8 * hh);
    kf[kk] = key < S ? a : v8{};
    vf[kk] = key < S ? b : v8{};
  }
  f32x16 dka[DT], dva[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) { dka[t] = f32x16{}; dva[t] = f32x16{}; }

  const int i_first = k0 / BQ;
  const int i_end = (S + BQ - 1) / BQ;
  const int wave_first_key = k0 + 32 * w;

  Tile64<D> qt, dt;
  float lreg = 0.f, ereg = 0.f;
  auto load_q = [&](int i) {
    qt.load(q + base, i * BQ, S);
    dt.load(dout + base, i * BQ, S);
    const int row = i * BQ + ((int)threadIdx.x & (BQ - 1));
    const int rc = row < S ? row : S - 1;
    const float lv = lsep[rc], ev = delp[rc];
    lreg = row < S ? lv * kLog2e : INFINITY;
    ereg = row < S ? ev : 0.f;
  };
  if (i_first < i_end) load_q(i_first);
  for (int i = i_first; i < i_end; ++i) {
    __syncthreads();
    qt.store_rows(Qs, RST);
    qt.store_cols(Qt, TST);
    dt.store_rows(Ds, RST);
    dt.store_cols(Dt, TST);
    if (threadIdx.x < BQ) { Ls[threadIdx.x] = lreg; Es[threadIdx.x] = ereg; }
    __syncthreads();
    const int qi0 = i * BQ;
    if (i + 1 < i_end) load_q(i + 1);
    if (qi0 + BQ - 1 < wave_first_key) continue;  // all rows above this wave's keys

    f32x16 s[2], dp[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) { s[mt] = f32x16{}; dp[mt] = f32x16{}; }
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        s[mt] = MM<T>::mma(ld16<v8>(Qs + (32 * mt + l32) * RST + kk * 16 + 8 * hh), kf[kk], s[mt]);
        dp[mt] = MM<T>::mma(ld16<v8>(Ds + (32 * mt + l32) * RST + kk * 16 + 8 * hh), vf[kk], dp[mt]);
      }
    const bool diag = qi0 < wave_first_key + 31;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int rr = 32 * mt + 8 * g + 4 * hh;  // first row of this 4-row group
        const float4 l4 = *reinterpret_cast<const float4*>(Ls + rr);
        const float4 e4 = *reinterpret_cast<const float4*>(Es + rr);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
        const float ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const int r = 4 * g + i4;
          float p = __builtin_amdgcn_exp2f(s[mt][r] * scale_log2 - lv[i4]);
          if (diag && key > qi0 + rr + i4) p = 0.f;
          s[mt][r] = p;
          dp[mt][r] = p * (dp[mt][r] - ev[i4]);
        }
      }
#pragma unroll
    for (int ms = 0; ms < BQ / 16; ++ms) {
      const v8 pb = pack8<T>(s[ms >> 1], 8 * (ms & 1));
      const v8 sb = pack8<T>(dp[ms >> 1], 8 * (ms & 1));
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const int off = toff(32 * t + l32, TST, ms * 16 + 8 * hh);
        dva[t] = MM<T>::mma(ld16<v8>(Dt + off), pb, dva[t]);
        dka[t] = MM<T>::mma(ld16<v8>(Qt + off), sb, dka[t]);
      }
    }
  }

  if (key < S) {
    uint16_t* dkp = dk + base + (int64_t)key * D;
    uint16_t* dvp = dv + base + (int64_t)key * D;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        *reinterpret_cast<uint2*>(dkp + 32 * t + 8 * g + 4 * hh) = pack4<T>(dka[t], 4 * g, scale);
        *reinterpret_cast<uint2*>(dvp + 32 * t + 8 * g + 4 * hh) = pack4<T>(dva[t], 4 * g, 1.0f);
      }
  }
}

// ------------------------------------------------------------------- dQ
template <typename T, int D>
__global__ __launch_bounds__(256, 1) void attn_dq_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, uint16_t* __restrict__ dq,
    int S, float scale, float scale_log2, int nqb) {
  using v8 = typename MM<T>::v8;
  constexpr int BM = 128, BN = 64;
  constexpr int KSTEPS = D / 16;
  constexpr int DT = D / 32;
  constexpr int RST = D + 8;
  constexpr int TST = BN + 8;
  __shared__ __align__(16) uint16_t Ks[BN * RST];
  __shared__ __align__(16) uint16_t Vs[BN * RST];
  __shared__ __align__(16) uint16_t Kt[D * TST];

  const int bh = blockIdx.y;
  const int qb = nqb - 1 - (int)blockIdx.x;
  const int q0 = qb * BM;
  const int lane = threadIdx.x & 63, w = wave_id();
  const int l32 = lane & 31, hh = lane >> 5;
  const int64_t base = (int64_t)bh * S * D;

  const int qrow = q0 + 32 * w + l32;
  const int qrc = qrow < S ? qrow : S - 1;
  v8 qf[KSTEPS], df[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) {
    const v8 a = ld16<v8>(q + base + (int64_t)qrc * D + kk * 16 + 8 * hh);
    const v8 b = ld16<v8>(dout + base + (int64_t)qrc * D + kk * 16 + 8 * hh);
    qf[kk] = qrow < S ? a : v8{};
    df[kk] = qrow < S ? b : v8{};
  }
  const float lv = lse[(int64_t)bh * S + qrc], ev = delta[(int64_t)bh * S + qrc];
  const float l2 = qrow < S ? lv * kLog2e : INFINITY;
  const float dl = qrow < S ? ev : 0.f;

  f32x16 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x16{};

  const int kv_end = min(S, q0 + BM);
  const int ntiles = (kv_end + BN - 1) / BN;
  const int wave_first_row = q0 + 32 * w;

  Tile64<D> kt, vt;
  kt.load(k + base, 0, S);
  vt.load(v + base, 0, S);
  for (int j = 0; j < ntiles; ++j) {
    __syncthreads();
    kt.store_rows(Ks, RST);
    kt.store_cols(Kt, TST);
    vt.store_rows(Vs, RST);
    __syncthreads();
    const int k0 = j * BN;
    if (j + 1 < ntiles) {
      kt.load(k + base, k0 + BN, S);
      vt.load(v + base, k0 + BN, S);
    }
    if (k0 > wave_first_row + 31) continue;

    f32x16 s[2], dp[2];
#pragma unroll
    for (int T2 = 0; T2 < 2; ++T2) { s[T2] = f32x16{}; dp[T2] = f32x16{}; }
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk)
#pragma unroll
      for (int T2 = 0; T2 < 2; ++T2) {
        s[T2] = MM<T>::mma(ld16<v8>(Ks + (32 * T2 + l32) * RST + kk * 16 + 8 * hh), qf[kk], s[T2]);
        dp[T2] = MM<T>::mma(ld16<v8>(Vs + (32 * T2 + l32) * RST + kk * 16 + 8 * hh), df[kk], dp[T2]);
      }
    const bool diag = k0 + BN - 1 > wave_first_row;
#pragma unroll
    for (int T2 = 0; T2 < 2; ++T2)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = __builtin_amdgcn_exp2f(s[T2][r] * scale_log2 - l2);
        if (diag) {
          const int key = k0 + 32 * T2 + (r >> 2) * 8 + 4 * hh + (r & 3);
          if (key > qrow) p = 0.f;
        }
        dp[T2][r] = p * (dp[T2][r] - dl);
      }
#pragma unroll
    for (int ms = 0; ms < BN / 16; ++ms) {
      const v8 sb = pack8<T>(dp[ms >> 1], 8 * (ms & 1));
#pragma unroll
      for (int t = 0; t < DT; ++t)
        acc[t] = MM<T>::mma(ld16<v8>(Kt + toff(32 * t + l32, TST, ms * 16 + 8 * hh)), sb, acc[t]);
    }
  }

  if (qrow < S) {
    uint16_t* op = dq + base + (int64_t)qrow * D;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<uint2*>(op + 32 * t + 8 * g + 4 * hh) = pack4<T>(acc[t], 4 * g, scale);
  }
}

// --------------------------------------------------------------- launchers
int check_attn(const char* what, int64_t B, int64_t H, int64_t S, int64_t D, int dtype) {
  if (B < 0 || H < 0 || S < 0) { set_error("%s: negative size", what); return 1; }
  if (D != 64 && D != 128) { set_error("%s: head_dim must be 64 or 128, got %lld", what, (long long)D); return 1; }
  if (dtype != EG_BF16 && dtype != EG_F16) { set_error("%s: dtype must be bf16 or fp16", what); return 1; }
  if (S > (int64_t)1 << 24 || B * H > 65535) { set_error("%s: size out of range", what); return 1; }
  return 0;
}

template <typename T, int D>
int attn_fwd_launch(const void* q, const void* k, const void* v, void* o, float* lse, int64_t BH,
                    int64_t S, float scale, hipStream_t st) {
  const int nqb = (int)((S + 127) / 128);
  hipLaunchKernelGGL((attn_fwd_kernel<T, D>), dim3((unsigned)nqb, (unsigned)BH), dim3(256), 0, st,
                     (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)o, lse,
                     (int)S, scale * kLog2e, nqb);
  return check_launch("eg_attn_fwd");
}

template <typename T, int D>
int attn_bwd_launch(const void* dout, const void* q, const void* k, const void* v, const void* o,
                    const float* lse, void* dq, void* dk, void* dv, float* delta, int64_t BH,
                    int64_t S, float scale, hipStream_t st) {
  const int64_t nrows = BH * S;
  const int64_t threads = nrows * (D / 8);
  hipLaunchKernelGGL((attn_delta_kernel<T, D>), dim3((unsigned)((threads + 255) / 256)), dim3(256),
                     0, st, (const uint16_t*)dout, (const uint16_t*)o, delta, nrows);
  if (int rc = check_launch("eg_attn_bwd(delta)")) return rc;
  const int nkb = (int)((S + 127) / 128);
  hipLaunchKernelGGL((attn_dkdv_kernel<T, D>), dim3((unsigned)nkb, (unsigned)BH), dim3(256), 0, st,
                     (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                     (const uint16_t*)dout, lse, delta, (uint16_t*)dk, (uint16_t*)dv, (int)S, scale,
                     scale * kLog2e, nkb);
  if (int rc = check_launch("eg_attn_bwd(dkdv)")) return rc;
  const int nqb = (int)((S + 127) / 128);
  hipLaunchKernelGGL((attn_dq_kernel<T, D>), dim3((unsigned)nqb, (unsigned)BH), dim3(256), 0, st,
                     (const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                     (const uint16_t*)dout, lse, delta, (uint16_t*)dq, (int)S, scale,
                     scale * kLog2e, nqb);
  return check_launch("eg_attn_bwd(dq)");
}

bool attn_aligned(std::initializer_list<const void*> ptrs) {
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  return true;
}

}  // namespace
}  // namespace eg

using namespace eg;

extern "C" size_t eg_attn_workspace_bytes(int64_t batch, int64_t heads, int64_t seq,
                                          int64_t head_dim) {
  (void)head_dim;
  if (batch <= 0 || heads <= 0 || seq <= 0) return 0;
  return (size_t)(batch * heads * seq) * sizeof(float);
}

extern "C" int eg_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                           int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                           float scale, int dtype, void* stream) {
  clear_error();
  if (check_attn("eg_attn_fwd", batch, heads, seq, head_dim, dtype)) return 1;
  if (batch == 0 || heads == 0 || seq == 0) return 0;
  if (!q || !k || !v || !o || !lse) { set_error("eg_attn_fwd: null pointer"); return 1; }
  if (!attn_aligned({q, k, v, o})) { set_error("eg_attn_fwd: tensors must be 16-byte aligned"); return 1; }
  hipStream_t st = as_stream(stream);
  const int64_t BH = batch * heads;
  if (dtype == EG_BF16)
    return head_dim == 128 ? attn_fwd_launch<bf16_t, 128>(q, k, v, o, lse, BH, seq, scale, st)
                           : attn_fwd_launch<bf16_t, 64>(q, k, v, o, lse, BH, seq, scale, st);
  return head_dim == 128 ? attn_fwd_launch<f16_t, 128>(q, k, v, o, lse, BH, seq, scale, st)
                         : attn_fwd_launch<f16_t, 64>(q, k, v, o, lse, BH, seq, scale, st);
}

extern "C" int eg_attn_bwd(const void* dout, const void* q, const void* k, const void* v,
                           const void* o, const float* lse, void* dq, void* dk, void* dv,
                           void* workspace, int64_t batch, int64_t heads, int64_t seq,
                           int64_t head_dim, float scale, int dtype, void* stream) {
  clear_error();
  if (check_attn("eg_attn_bwd", batch, heads, seq, head_dim, dtype)) return 1;
  if (batch == 0 || heads == 0 || seq == 0) return 0;
  if (!dout || !q || !k || !v || !o || !lse || !dq || !dk || !dv || !workspace) {
    set_error("eg_attn_bwd: null pointer");
    return 1;
  }
  if (!attn_aligned({dout, q, k, v, o, dq, dk, dv})) {
    set_error("eg_attn_bwd: tensors must be 16-byte aligned");
    return 1;
  }
  hipStream_t st = as_stream(stream);
  const int64_t BH = batch * heads;
  float* delta = (float*)workspace;
  if (dtype == EG_BF16)
    return head_dim == 128
               ? attn_bwd_launch<bf16_t, 128>(dout, q, k, v, o, lse, dq, dk, dv, delta, BH, seq, scale, st)
               : attn_bwd_launch<bf16_t, 64>(dout, q, k, v, o, lse, dq, dk, dv, delta, BH, seq, scale, st);
  return head_dim == 128
             ? attn_bwd_launch<f16_t, 128>(dout, q, k, v, o, lse, dq, dk, dv, delta, BH, seq, scale, st)
             : attn_bwd_launch<f16_t, 64>(dout, q, k, v, o, lse, dq, dk, dv, delta, BH, seq, scale, st);
}
