// vkv_refattn.hip -- quantized attention with the reference's own
// arithmetic, in three passes over any query length, mask, group size and
// float dtype:
//
//   1. scores:  q (times the dtype-rounded scale, rounded to the dtype) .
//      dequant(K), accumulated in fp32 and stored in the query dtype, as
//      quantizedMM returns T (Libraries/MLXLMCommon/KVCache.swift:1945-1949);
//      the mask as :1951-1975 applies it (causal / bool: where(mask, s,
//      finfo.min); additive: s + mask, in T for a mask of T, promoted to
//      f32 for an f32 mask);
//   2. softmax(scores, axis: -1) with precise: false (:1982,
//      Source/MLX/Ops.swift:2702-2710): the Metal kernels' default
//      AccT = T (Source/Cmlx/mlx-generated/metal/softmax.h:10, :100), i.e.
//      exponentials, partial sums and the normaliser rounded to T, with the
//      grouping of softmax_single_row (:10-98: 4 consecutive keys per
//      thread, 32-thread simd sums, then their sum) for rows of up to 4096
//      keys and of softmax_looped (:100-190: 1024 threads, each a running
//      (max, sum) rescaled at every round) above; weights stored in T.  An
//      f32 additive mask keeps the row in f32 (fp32 softmax, f32 weights);
//   3. P.V: the stored weights times dequant(V), fp32 accumulation, the
//      output rounded to T.
// With 16 or more query tokens the reference's quantized matmul runs its
// tiled path, which dequantizes K and V tiles to T first
// (quantized.h:568-576, :686-713): deq_round rounds them the same way.
//
// The softmax pass mirrors that grouping exactly and does its sums in
// fp64 (each partial sum rounded as the AccT arithmetic rounds it), so
// from the same stored scores it produces the same weights bit for bit as
// the oracle's restatement.  The order of the fp32 additions inside one
// Metal simd_sum is the hardware's and not in the tree; fp64 sums of at
// most 32 dtype-rounded terms are exact in practice, so any order agrees.
//
// This path trades speed for the reference's rounding: the score buffer is
// written and read back, and the softmax is its own pass.  One-token decode
// over paged bf16 4/8-bit views runs passes 1 and 3 on matrix cores
// instead (qdecode_kernel's score and weight modes, vkv_decode.hip).
#include "vkv_device.h"
#include "vkv_internal.h"
#include "vkv_kvread.h"

#include <algorithm>

namespace vkv {

namespace {

constexpr int kRefTile = 64;    // tokens per score / P.V tile
constexpr int kRefRows = 16;    // query rows per block of the score and P.V passes
constexpr int kSoftmaxThreads = 1024;
constexpr int kSoftmaxReads = 4;
constexpr int kSoftmaxLoopedLimit = 4096;

__device__ __forceinline__ int64_t row_len(const KVSrc& kv, int64_t b) {
  return kv.seq_lens ? kv.seq_lens[b] : kv.T;
}

// x rounded to float, then to dtype DT (0 f32, 1 f16, 2 bf16): the AccT
// arithmetic's rounding of an fp64 value.
template <int DT>
__device__ __forceinline__ double rnd_d(double x) {
  const float f = static_cast<float>(x);
  if constexpr (DT == kF16) return static_cast<double>(round_to<kF16>(f));
  else if constexpr (DT == kBF16) return static_cast<double>(round_to<kBF16>(f));
  else return static_cast<double>(f);
}
// (not inlined: the fp64 exp is the rare path of t_exp_fast, and inlined
// at every call it grew the softmax kernel past the instruction cache)
template <int DT>
__device__ __attribute__((noinline)) double t_exp(double x) { return rnd_d<DT>(exp(x)); }

template <int DT>
__device__ __forceinline__ double type_max_d() {
  return DT == kF16 ? 65504.0 : DT == kBF16 ? 3.38953139e38 : 3.402823466e38;
}

// Score / weight storage: float, or bf16 bit patterns (the matrix-core
// decode path's bf16 rows).
template <typename S> struct Store;
template <> struct Store<float> {
  __device__ __forceinline__ static double get(const float* p, int64_t i) { return p[i]; }
  __device__ __forceinline__ static void put(float* p, int64_t i, double v) { p[i] = static_cast<float>(v); }
};
template <> struct Store<uint16_t> {
  __device__ __forceinline__ static double get(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
  __device__ __forceinline__ static void put(uint16_t* p, int64_t i, double v) {
    p[i] = f32_to_bf16(static_cast<float>(v));
  }
};

}  // namespace

// ---- pass 1: scores.  Workgroup = one (64-token tile, kv head, batch
// row); the tile's keys are dequantized into LDS once, then every query row
// of the kv head (rep heads x the batch of query positions) is scored
// against them, 16 rows at a time.
template <int DT, int BITS>
__global__ void __launch_bounds__(256) ref_scores_kernel(RefArgs r) {
  using E = Elem<DT>;
  const AttnArgs& a = r.a;
  extern __shared__ float smem[];
  __shared__ TokLoc loc[kRefTile];
  const int D = a.D, tid = threadIdx.x;
  const int hk = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int64_t T = row_len(a.kv, b);
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kRefTile;
  if (t0 >= T) return;
  const int nt = static_cast<int>(min<int64_t>(kRefTile, T - t0));
  float* kt = smem;                         // [kRefTile][D + 1]
  float* qs = smem + kRefTile * (D + 1);    // [kRefRows][D]
  if (tid < nt) loc[tid] = locate(a.kv, b, t0 + tid);
  __syncthreads();
  for (int i = tid; i < nt * D; i += 256) {
    const int t = i / D, d = i % D;
    const float v = kv_at<DT, BITS>(a.kv, loc[t], hk, d, 0, r.group);
    kt[t * (D + 1) + d] = r.deq_round ? round_to<DT>(v) : v;
  }
  const int rep = a.Hq / a.Hkv, nl = r.nl, nrows = rep * nl;
  const float scale_t = round_to<DT>(a.scale);
  const int tt = tid & 63, rg = tid >> 6;
  const float lowest = -E::kMax;
  for (int rb = 0; rb < nrows; rb += kRefRows) {
    __syncthreads();  // the key tile is complete; the previous rows are done
    for (int i = tid; i < kRefRows * D; i += 256) {
      const int ri = rb + i / D, d = i % D;
      float v = 0.0f;
      if (ri < nrows) {
        const int h = hk * rep + ri / nl, l = r.l0 + ri % nl;
        const float qv = E::load(static_cast<const typename E::T*>(a.q) + b * a.q_sb + h * a.q_sh +
                                 static_cast<int64_t>(l) * a.q_sl + d);
        v = round_to<DT>(qv * scale_t);
      }
      qs[i] = v;
    }
    __syncthreads();
    if (tt >= nt) continue;
    const float* kr = kt + tt * (D + 1);
    const int64_t t = t0 + tt;
    for (int k = rg; k < kRefRows; k += 4) {
      const int ri = rb + k;
      if (ri >= nrows) break;
      const float* qr = qs + k * D;
      float acc = 0.0f;
      for (int d = 0; d < D; d++) acc = fmaf(qr[d], kr[d], acc);
      const int h = hk * rep + ri / nl, li = ri % nl, l = r.l0 + li;
      float s = round_to<DT>(acc);
      bool vis = true;
      if (a.mask_mode == 1) {
        vis = t <= T - a.L + l;
      } else if (a.mask_mode >= 2) {
        const int64_t mo = b * a.m_sb + h * a.m_sh + static_cast<int64_t>(l) * a.m_sl + t * a.m_st;
        if (a.mask_mode == 2) {
          vis = static_cast<const uint8_t*>(a.mask)[mo] != 0;
        } else {
          const float add = load_f32(a.mask, a.mask_dtype, mo);
          s = a.mask_dtype == DT ? round_to<DT>(s + add) : s + add;
        }
      }
      if (!vis) s = lowest;
      r.sc[((b * a.Hq + h) * nl + li) * r.tpad + t] = s;
    }
  }
}

// ---- pass 2: the reference softmax of one row, in place over the stored
// scores.  A workgroup of 256 threads plays the reference's 1024: thread
// lid is threads lid + 256 k (k = 0..3), so the reference's grouping (4
// keys per thread, simd groups of 32 threads) is kept; each simd group's
// 32 threads are one half-wave of ours.  acc_dt: the AccT dtype, or -1 for
// the fp32 arithmetic of an f32-promoted row; w_dt: the weights' dtype.
// The fp64 sums of dtype-rounded terms are exact, so their order (here a
// half-wave butterfly) does not change them.
constexpr int kSmThreads = 256;
constexpr int kSmVirtual = kSoftmaxThreads / kSmThreads;  // reference threads per thread

// exp of a dtype value x, rounded as rnd_d rounds it (fp64 exp, to float,
// to the dtype).  Below the dtype's underflow (exp(x) under half its
// smallest subnormal: x < -25 ln 2 for f16, x < -134 ln 2 for bf16) that is
// 0.  Otherwise the f32 exp decides it unless its result sits within 16
// float ulps of a dtype rounding midpoint (or under the dtype's normal
// range), where the fp64 exp does.
template <int DT>
__device__ __forceinline__ double t_exp_fast(double x) {
  if constexpr (DT == kBF16) {
    if (x < -93.0) return 0.0;
    const float e = expf(static_cast<float>(x));
    const uint32_t lo = __float_as_uint(e) & 0xFFFFu;
    if (e >= 1.2e-38f && (lo + 16u < 0x8000u || lo > 0x8000u + 16u))
      return static_cast<double>(round_to<kBF16>(e));
  } else if constexpr (DT == kF16) {
    if (x < -17.5) return 0.0;
    const float e = expf(static_cast<float>(x));
    const uint32_t lo = __float_as_uint(e) & 0x1FFFu;
    if (e >= 6.2e-5f && (lo + 16u < 0x1000u || lo > 0x1000u + 16u))
      return static_cast<double>(round_to<kF16>(e));
  }
  return t_exp<DT>(x);
}

__device__ __forceinline__ double half_sum(double x) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) x += __shfl_xor(x, o, 32);
  return x;
}
__device__ __forceinline__ double half_max(double x) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) x = fmax(x, __shfl_xor(x, o, 32));
  return x;
}

// Rows are staged through LDS in windows of up to kSmWindow scores (all of a
// window's loads in flight at once); a row that fits one window stays there
// for the final pass.
constexpr int kSmWindow = 16384;
// The window of a launch: its longest row rounded up to whole rounds of the
// looped softmax (4096 scores), at most kSmWindow, so short rows take less
// LDS and more of them run on a CU.
inline int sm_window(int64_t max_len) {
  constexpr int kRound = kSoftmaxReads * kSoftmaxThreads;
  const int64_t w = (std::max<int64_t>(max_len, 1) + kRound - 1) / kRound * kRound;
  return static_cast<int>(std::min<int64_t>(w, kSmWindow));
}

// The LDS copy of a window of a score row.  Scores stored in a 16-bit
// dtype (bf16 rows, or f32 rows holding values rounded to bf16 / f16 for
// that dtype's softmax) are kept as their 16-bit patterns: exact, and half
// the LDS of floats, so twice the workgroups a CU.  Rows of f32 arithmetic
// stay floats.
template <typename S, int ACC> struct SmLds {
  static constexpr bool kHalf = sizeof(S) == 2 || ACC == kF16 || ACC == kBF16;
  static constexpr int kDt = sizeof(S) == 2 ? kBF16 : ACC;  // the 16-bit dtype
  using T = typename std::conditional<kHalf, uint16_t, float>::type;
  __device__ __forceinline__ static T put(S x) {
    if constexpr (!kHalf) return x;
    else if constexpr (sizeof(S) == 2) return x;
    else if constexpr (kDt == kF16) return f32_to_f16(x);
    else return f32_to_bf16(x);
  }
  __device__ __forceinline__ static double val(T x) {
    if constexpr (!kHalf) return x;
    else if constexpr (kDt == kF16) return f16_to_f32(x);
    else return bf16_to_f32(x);
  }
};

template <typename S, int ACC>
__device__ __forceinline__ void sm_stage(const S* p, int64_t w0, int wlen,
                                         typename SmLds<S, ACC>::T* buf, int lid) {
  using L = SmLds<S, ACC>;
  constexpr int U = 16;
  for (int i0 = 0; i0 < wlen; i0 += U * kSmThreads) {
    typename L::T v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = i0 + u * kSmThreads + lid;
      v[u] = i < wlen ? L::put(p[w0 + i]) : typename L::T{};
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = i0 + u * kSmThreads + lid;
      if (i < wlen) buf[i] = v[u];
    }
  }
}

// win: the LDS window (sm_window of the launch's longest row), in the
// dynamic LDS the launch passes.
template <typename S, int ACC>
__global__ void __launch_bounds__(kSmThreads) ref_softmax_kernel(S* sc, int64_t tpad,
                                                                 const int32_t* seq_lens,
                                                                 int32_t T_all, int64_t per_b,
                                                                 int win) {
  // ACC: the AccT dtype, or -1 for an f32-promoted row (fp32 arithmetic,
  // f32 weights)
  constexpr int dt = ACC < 0 ? kF32 : ACC;
  using St = Store<S>;
  using L = SmLds<S, ACC>;
  extern __shared__ __attribute__((aligned(16))) unsigned char sm_win[];
  typename L::T* buf = reinterpret_cast<typename L::T*>(sm_win);
  __shared__ double red[kSmThreads / 64];
  __shared__ double simd_s[kSoftmaxThreads / 32], simd_m[kSoftmaxThreads / 32];
  __shared__ double bcast[2];
  const int64_t row = blockIdx.x;
  const int64_t T = seq_lens ? seq_lens[row / per_b] : T_all;
  if (T <= 0) return;
  S* p = sc + row * tpad;
  const int lid = threadIdx.x, lane = lid & 63, wv = lid >> 6;
  const bool resident = T <= win;  // the whole row stays in LDS
  // score t: from LDS when the row is resident
  auto score = [&](int64_t t) __attribute__((always_inline)) {
    return resident ? L::val(buf[t]) : St::get(p, t);
  };

  // row max (of stored values: exact in any order), window by window
  double mx = -INFINITY;
  for (int64_t w0 = 0; w0 < T; w0 += win) {
    const int wlen = static_cast<int>(min<int64_t>(win, T - w0));
    if (w0 > 0) __syncthreads();
    sm_stage<S, ACC>(p, w0, wlen, buf, lid);
    __syncthreads();
    for (int i = lid; i < wlen; i += kSmThreads) mx = fmax(mx, L::val(buf[i]));
  }
  mx = half_max(mx);
  mx = fmax(mx, __shfl_xor(mx, 32));
  if (lane == 0) red[wv] = mx;
  __syncthreads();
  mx = fmax(fmax(red[0], red[1]), fmax(red[2], red[3]));
  __syncthreads();

  if constexpr (ACC < 0) {
    // fp32 arithmetic: exp of the f32 difference, summed, one reciprocal
    double sum = 0.0;
    for (int64_t t = lid; t < T; t += kSmThreads)
      sum += static_cast<double>(static_cast<float>(exp(static_cast<double>(static_cast<float>(score(t) - mx)))));
    sum = half_sum(sum);
    sum += __shfl_xor(sum, 32);
    if (lane == 0) red[wv] = sum;
    __syncthreads();
    const double tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float rr = static_cast<float>(1.0 / static_cast<double>(static_cast<float>(tot)));
    for (int64_t t = lid; t < T; t += kSmThreads) {
      const float e = static_cast<float>(exp(static_cast<double>(static_cast<float>(score(t) - mx))));
      St::put(p, t, rnd_d<kF32>(static_cast<double>(e * rr)));
    }
    return;
  }
  if (T <= kSoftmaxLoopedLimit) {
    // softmax_single_row: reference thread v = lid + 256 k owns keys 4v .. 4v + 3
    double e[kSmVirtual][kSoftmaxReads];
#pragma unroll
    for (int k = 0; k < kSmVirtual; k++) {
      double thr = 0.0;
#pragma unroll
      for (int i = 0; i < kSoftmaxReads; i++) {
        const int64_t t = static_cast<int64_t>(kSoftmaxReads) * (lid + kSmThreads * k) + i;
        e[k][i] = t < T ? t_exp_fast<dt>(rnd_d<dt>(L::val(buf[t]) - mx)) : 0.0;
        if (t < T) thr = rnd_d<dt>(thr + e[k][i]);
      }
      // simd group (lid + 256 k) / 32: this half-wave
      const double sg = half_sum(thr);
      if ((lid & 31) == 0) simd_s[(lid >> 5) + (kSmThreads / 32) * k] = rnd_d<dt>(sg);
    }
    __syncthreads();
    if (wv == 0) {
      const int nsimd = static_cast<int>((T + 127) / 128);
      double tot = lane < 32 && lane < nsimd ? simd_s[lane] : 0.0;
      tot = half_sum(tot);
      if (lane == 0) bcast[0] = rnd_d<dt>(1.0 / rnd_d<dt>(tot));
    }
    __syncthreads();
    const double rr = bcast[0];
#pragma unroll
    for (int k = 0; k < kSmVirtual; k++)
#pragma unroll
      for (int i = 0; i < kSoftmaxReads; i++) {
        const int64_t t = static_cast<int64_t>(kSoftmaxReads) * (lid + kSmThreads * k) + i;
        if (t < T) St::put(p, t, rnd_d<dt>(e[k][i] * rr));
      }
    return;
  }
  // softmax_looped: reference thread v keeps a running (max, sum) over keys
  // 4v + 4096 r + i, rescaled at every round; the rounds go window by window
  const double fmin = -type_max_d<dt>();
  const int64_t stride = static_cast<int64_t>(kSoftmaxReads) * kSoftmaxThreads;
  const int64_t rounds = (T + stride - 1) / stride;
  const int rounds_per_window = win / (kSoftmaxReads * kSoftmaxThreads);
  double m[kSmVirtual], n[kSmVirtual];
#pragma unroll
  for (int k = 0; k < kSmVirtual; k++) {
    m[k] = fmin;
    n[k] = 0.0;
  }
  for (int64_t rd0 = 0; rd0 < rounds; rd0 += rounds_per_window) {
    const int64_t w0 = rd0 * stride;
    const int wlen = static_cast<int>(min<int64_t>(win, T - w0));
    if (!resident) {
      __syncthreads();
      sm_stage<S, ACC>(p, w0, wlen, buf, lid);
      __syncthreads();
    }
    const int64_t rd1 = min<int64_t>(rounds, rd0 + rounds_per_window);
    for (int64_t rd = rd0; rd < rd1; rd++) {
#pragma unroll
      for (int k = 0; k < kSmVirtual; k++) {
        const int64_t off = rd * stride + static_cast<int64_t>(lid + kSmThreads * k) * kSoftmaxReads;
        double v[kSoftmaxReads];
        const double prev = m[k];
#pragma unroll
        for (int i = 0; i < kSoftmaxReads; i++) {
          v[i] = off + i < T ? L::val(buf[off + i - w0]) : -INFINITY;
          m[k] = v[i] > m[k] ? v[i] : m[k];
        }
        n[k] = rnd_d<dt>(n[k] * t_exp_fast<dt>(rnd_d<dt>(prev - m[k])));
#pragma unroll
        for (int i = 0; i < kSoftmaxReads; i++) n[k] = rnd_d<dt>(n[k] + t_exp_fast<dt>(rnd_d<dt>(v[i] - m[k])));
      }
    }
  }
#pragma unroll
  for (int k = 0; k < kSmVirtual; k++) {
    // simd group (lid + 256 k) / 32: its max, then the rescaled sums
    const double mg = half_max(m[k]);
    const double acc = half_sum(rnd_d<dt>(n[k] * t_exp_fast<dt>(rnd_d<dt>(m[k] - mg))));
    if ((lid & 31) == 0) {
      simd_m[(lid >> 5) + (kSmThreads / 32) * k] = mg;
      simd_s[(lid >> 5) + (kSmThreads / 32) * k] = rnd_d<dt>(acc);
    }
  }
  __syncthreads();
  if (wv == 0) {
    const double sm = lane < 32 ? simd_m[lane] : fmin;
    const double gmax = half_max(sm);
    double tot = lane < 32 ? rnd_d<dt>(simd_s[lane] * t_exp_fast<dt>(rnd_d<dt>(sm - gmax))) : 0.0;
    tot = half_sum(tot);
    if (lane == 0) {
      bcast[0] = gmax;
      bcast[1] = rnd_d<dt>(1.0 / rnd_d<dt>(tot));
    }
  }
  __syncthreads();
  const double gmax = bcast[0], rr = bcast[1];
  if (resident) {
    for (int64_t t = lid; t < T; t += kSmThreads)
      St::put(p, t, rnd_d<dt>(t_exp_fast<dt>(rnd_d<dt>(L::val(buf[t]) - gmax)) * rr));
    return;
  }
  for (int64_t w0 = 0; w0 < T; w0 += win) {
    const int wlen = static_cast<int>(min<int64_t>(win, T - w0));
    __syncthreads();
    sm_stage<S, ACC>(p, w0, wlen, buf, lid);
    __syncthreads();
    for (int i = lid; i < wlen; i += kSmThreads)
      St::put(p, w0 + i, rnd_d<dt>(t_exp_fast<dt>(rnd_d<dt>(L::val(buf[i]) - gmax)) * rr));
  }
}

// ---- pass 3: out = sum_t w_t dequant(v_t).  Workgroup = (token part, kv
// head x 16-row block, batch row); value tiles dequantized into LDS, each
// thread owns up to 16 (row, dim) outputs; parts are summed in order by
// ref_merge_kernel.
template <int DT, int BITS>
__global__ void __launch_bounds__(256) ref_pv_kernel(RefArgs r) {
  using E = Elem<DT>;
  const AttnArgs& a = r.a;
  extern __shared__ float smem[];
  __shared__ TokLoc loc[kRefTile];
  __shared__ float wt[kRefRows][kRefTile];
  const int Dv = a.Dv, tid = threadIdx.x;
  const int rep = a.Hq / a.Hkv, nl = r.nl, nrows = rep * nl;
  const int nrb = (nrows + kRefRows - 1) / kRefRows;
  const int hk = blockIdx.y / nrb, rb = (blockIdx.y % nrb) * kRefRows;
  const int64_t b = blockIdx.z;
  const int part = blockIdx.x;
  const int64_t T = row_len(a.kv, b);
  const int64_t tb = static_cast<int64_t>(part) * r.part_tokens;
  const int64_t te = min<int64_t>(T, tb + r.part_tokens);
  float* vt = smem;  // [kRefTile][Dv]
  constexpr int kOut = kRefRows * 256 / 256;  // outputs per thread at Dv <= 256
  float acc[kOut];
#pragma unroll
  for (int k = 0; k < kOut; k++) acc[k] = 0.0f;
  const int nout = kRefRows * Dv;
  for (int64_t t0 = tb; t0 < te; t0 += kRefTile) {
    const int nt = static_cast<int>(min<int64_t>(kRefTile, te - t0));
    __syncthreads();  // the previous tile is consumed
    if (tid < nt) loc[tid] = locate(a.kv, b, t0 + tid);
    for (int i = tid; i < kRefRows * kRefTile; i += 256) {
      const int k = i / kRefTile, t = i % kRefTile;
      const int ri = rb + k;
      float w = 0.0f;
      if (ri < nrows && t < nt) {
        const int h = hk * rep + ri / nl, li = ri % nl;
        w = r.sc[((b * a.Hq + h) * nl + li) * r.tpad + t0 + t];
      }
      wt[k][t] = w;
    }
    __syncthreads();
    for (int i = tid; i < nt * Dv; i += 256) {
      const int t = i / Dv, d = i % Dv;
      const float v = kv_at<DT, BITS>(a.kv, loc[t], hk, d, 1, r.group);
      vt[t * Dv + d] = r.deq_round ? round_to<DT>(v) : v;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kOut; k++) {
      const int o = tid + 256 * k;
      if (o >= nout) break;
      const int row = o / Dv, d = o % Dv;
      float s = acc[k];
      for (int t = 0; t < nt; t++) s = fmaf(wt[row][t], vt[t * Dv + d], s);
      acc[k] = s;
    }
  }
#pragma unroll
  for (int k = 0; k < kOut; k++) {
    const int o = tid + 256 * k;
    if (o >= nout) break;
    const int row = o / Dv, d = o % Dv;
    const int ri = rb + row;
    if (ri >= nrows) continue;
    const int h = hk * rep + ri / nl, li = ri % nl;
    const int64_t ridx = (b * a.Hq + h) * nl + li;
    if (r.n_parts == 1) {
      static_cast<typename E::T*>(a.out)[b * a.o_sb + h * a.o_sh +
                                         static_cast<int64_t>(r.l0 + li) * a.o_sl + d] = E::from_f32(acc[k]);
    } else {
      r.ws[(static_cast<int64_t>(part) * r.n_rows + ridx) * Dv + d] = acc[k];
    }
  }
}

// The parts' sums, added in part order.
template <int DT>
__global__ void __launch_bounds__(256) ref_merge_kernel(RefArgs r) {
  using E = Elem<DT>;
  const AttnArgs& a = r.a;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= r.n_rows * a.Dv) return;
  const int64_t ridx = i / a.Dv;
  const int d = static_cast<int>(i % a.Dv);
  float s = 0.0f;
  for (int p = 0; p < r.n_parts; p++) s += r.ws[(static_cast<int64_t>(p) * r.n_rows + ridx) * a.Dv + d];
  const int nl = r.nl;
  const int64_t li = ridx % nl, bh = ridx / nl, h = bh % a.Hq, b = bh / a.Hq;
  static_cast<typename E::T*>(a.out)[b * a.o_sb + h * a.o_sh + (r.l0 + li) * a.o_sl + d] = E::from_f32(s);
}

// ---------------------------------------------------------------- host

size_t ref_scores_lds(int D) { return sizeof(float) * (kRefTile * (D + 1) + kRefRows * D); }
size_t ref_pv_lds(int Dv) { return sizeof(float) * kRefTile * Dv; }

int ref_part_tokens(int64_t B, int Hkv, int nrows, int64_t T, int* n_parts) {
  const int64_t nrb = (nrows + kRefRows - 1) / kRefRows;
  const int64_t groups = std::max<int64_t>(1, B * Hkv * nrb);
  int64_t parts = std::max<int64_t>(1, (2048 + groups - 1) / groups);
  parts = std::min<int64_t>(parts, std::max<int64_t>(1, (T + kRefTile - 1) / kRefTile));
  int64_t pt = (std::max<int64_t>(T, 1) + parts - 1) / parts;
  pt = (pt + kRefTile - 1) / kRefTile * kRefTile;
  *n_parts = static_cast<int>(std::max<int64_t>(1, (T + pt - 1) / pt));
  return static_cast<int>(pt);
}

// One workgroup a row; the LDS window sized to the launch's longest row
// (max_len), in dynamic LDS.
template <typename S, int ACC>
static void launch_softmax(dim3 rows, S* sc, int64_t tpad, const int32_t* seq_lens,
                           int32_t max_len, int64_t per_b, hipStream_t st) {
  using T = typename SmLds<S, ACC>::T;
  static const bool lds_ok = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&ref_softmax_kernel<S, ACC>),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(kSmWindow * sizeof(T))) == hipSuccess;
  }();
  VKV_CHECK(lds_ok, "cannot raise the softmax kernel's LDS limit");
  const int win = sm_window(max_len);
  hipLaunchKernelGGL((ref_softmax_kernel<S, ACC>), rows, dim3(kSmThreads), win * sizeof(T), st, sc,
                     tpad, seq_lens, max_len, per_b, win);
}

template <int DT, int BITS>
static void ref_launch_dt(const RefArgs& r, int64_t B, hipStream_t st) {
  const AttnArgs& a = r.a;
  const int rep = a.Hq / a.Hkv, nrows = rep * r.nl;
  const int64_t T = a.kv.T;
  const dim3 gs(static_cast<unsigned>((std::max<int64_t>(T, 1) + kRefTile - 1) / kRefTile),
                static_cast<unsigned>(a.Hkv), static_cast<unsigned>(B));
  // above 64 KB of dynamic LDS (head dims over ~200) the kernel must ask
  static const bool lds_ok = [] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&ref_scores_kernel<DT, BITS>),
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(ref_scores_lds(kMaxRefD))) == hipSuccess;
  }();
  VKV_CHECK(lds_ok, "cannot raise the score kernel's LDS limit");
  hipLaunchKernelGGL((ref_scores_kernel<DT, BITS>), gs, dim3(256), ref_scores_lds(a.D), st, r);
  VKV_HIP(hipGetLastError());
  const dim3 rows(static_cast<unsigned>(B * a.Hq * r.nl));
  const int64_t per_b = static_cast<int64_t>(a.Hq) * r.nl;
  if (r.score_f32)
    launch_softmax<float, -1>(rows, r.sc, r.tpad, a.kv.seq_lens, a.kv.T, per_b, st);
  else
    launch_softmax<float, DT>(rows, r.sc, r.tpad, a.kv.seq_lens, a.kv.T, per_b, st);
  VKV_HIP(hipGetLastError());
  const int nrb = (nrows + kRefRows - 1) / kRefRows;
  const dim3 gp(static_cast<unsigned>(r.n_parts), static_cast<unsigned>(a.Hkv * nrb),
                static_cast<unsigned>(B));
  hipLaunchKernelGGL((ref_pv_kernel<DT, BITS>), gp, dim3(256), ref_pv_lds(a.Dv), st, r);
  VKV_HIP(hipGetLastError());
  if (r.n_parts > 1) {
    const int64_t n = r.n_rows * a.Dv;
    hipLaunchKernelGGL((ref_merge_kernel<DT>), dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                       st, r);
    VKV_HIP(hipGetLastError());
  }
}

template <int DT>
static void ref_launch_bits(const RefArgs& r, int64_t B, hipStream_t st) {
  if (r.bits == 4) ref_launch_dt<DT, 4>(r, B, st);
  else if (r.bits == 8) ref_launch_dt<DT, 8>(r, B, st);
  else throw Error("reference-arithmetic attention needs an affine 4- or 8-bit cache");
}

void launch_ref_attention(int dtype, const RefArgs& r, int64_t B, hipStream_t st) {
  VKV_CHECK(r.a.D <= kMaxRefD && r.a.Dv <= kMaxRefD, "head dims above 256 are not supported here");
  VKV_CHECK(r.a.Hq % r.a.Hkv == 0, "query heads must be a multiple of kv heads");
  switch (dtype) {
    case kF32: ref_launch_bits<kF32>(r, B, st); break;
    case kF16: ref_launch_bits<kF16>(r, B, st); break;
    case kBF16: ref_launch_bits<kBF16>(r, B, st); break;
    default: throw Error("unsupported dtype");
  }
}

// The reference softmax over bf16 score rows (the matrix-core decode
// path): rows of seq_lens[row / per_b] (or T) scores, tpad apart.
void launch_ref_softmax_bf16(uint16_t* sc, int64_t rows, int64_t tpad, const int32_t* seq_lens,
                             int32_t T, int64_t per_b, hipStream_t st) {
  if (rows <= 0) return;
  launch_softmax<uint16_t, kBF16>(dim3(static_cast<unsigned>(rows)), sc, tpad, seq_lens, T, per_b,
                                  st);
  VKV_HIP(hipGetLastError());
}

}  // namespace vkv
