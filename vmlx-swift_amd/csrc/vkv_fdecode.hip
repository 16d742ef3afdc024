// vkv_fdecode.hip -- decode attention (one query token per row) over dense
// float K/V: the MLXFast SDPA of KVCacheSimple / RotatingKVCache decode
// steps (sdpa_vector.h:15-177, MLXFast.swift:173-218).
//
// Semantics as the generic attention kernel's MLXFast mode: queries scaled
// in fp32, scores and the probability-weighted sum in fp32, masked keys
// skipped (a bool mask) or offset (an additive f32 mask), an empty row
// yields zeros; split partials are merged by attn_combine_kernel as
// sdpa_vector_2pass_2 merges them (sdpa_vector.h:320-394).
//
// Layout.  One wave per workgroup owns a (row, kv head, head group, token
// range) and walks it 32 tokens at a time:
//   * scores, bf16 / f16 K/V: on matrix cores, S^T (16 tokens x 16 columns,
//     the group's REP <= 8 heads) = K (A operands: lane (m, g) loads dims
//     32 s + 8 g .. + 7 of token m of a 16-token tile, 16 bytes straight
//     from memory) . Q^T (B operands: the raw queries in registers), one
//     16x16x32 MFMA per tile and 32 dims; the fp32 scores are then scaled
//     (the reference scales the queries first: the same fp32 arithmetic up
//     to summation order).  The max and sum of a head reduce over the four
//     lanes that hold it and reach every lane through readlane (config 4's
//     window layer: 16.0 -> 12.1 us; config 1's step 17.8 -> 16.1 us);
//   * scores, f32 K/V: lanes t and t + 32 own token t, each taking half of
//     its key row with 16-byte loads (every byte of a row used), against the
//     queries of the group's REP heads in LDS; one lane swap adds the
//     halves.  Two lanes per token give a launch twice the waves of one
//     lane per token for the same bytes (a 33.6 MB D = 256 decode: 14.9 ->
//     12.3 us).
//   * online softmax per head over the 32 scores (DPP reductions within
//     each half-wave), the probabilities into LDS;
//   * values: lanes own 16-byte runs of a value row, D/8 (bf16/f16) or D/4
//     (f32) lanes per row, so every load instruction reads whole rows;
//     the lanes that share a run sum their tokens at the end.
// The value contraction stays on the vector ALUs (at REP <= 8 query heads
// per kv head about one FMA per KV byte); on matrix cores its value rows
// would have to be transposed through LDS.
//
// Split merge.  With counters (one per (row, kv head, head group)) the
// parts merge inside the launch: each part stores its (o, max, sum)
// partial with device-coherent stores (relaxed agent-scope atomics, which
// write through to the level every XCD reads), waits for them to complete,
// and counts itself in; the part that counts last reads every partial back
// with device-coherent loads, merges them as sdpa_vector_2pass_2 does and
// writes the output, then zeroes the counter for the next launch.  No
// fence writes back or invalidates an L2, and a part has no loads in
// flight when it waits for its stores.  Without counters the partials go
// to attn_combine_kernel (a launch of its own).
#include <algorithm>

#include "vkv_device.h"
#include <hip/hip_ext.h>
#include "vkv_internal.h"

namespace vkv {

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;

// 16x16x32 MFMA on 16-bit operands of the cache dtype
template <int DT>
__device__ __forceinline__ f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  if constexpr (DT == kF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Tokens per step: two lanes per token, each scoring half of the dims.
constexpr int kStep = 32;

// 16 loaded bytes -> VEC floats
template <int DT>
__device__ __forceinline__ void unpack16(const u32x4_t& w, float* out) {
  if constexpr (DT == kF32) {
#pragma unroll
    for (int e = 0; e < 4; e++) out[e] = __uint_as_float(w[e]);
  } else if constexpr (DT == kBF16) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      out[2 * e] = __uint_as_float(w[e] << 16);
      out[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      out[2 * e] = f16_to_f32(static_cast<uint16_t>(w[e] & 0xFFFFu));
      out[2 * e + 1] = f16_to_f32(static_cast<uint16_t>(w[e] >> 16));
    }
  }
}

// Cross-lane moves without an LDS round trip where one exists: DPP inside
// rows of 16 lanes, the swizzle for partners 8 and 16 lanes away (within
// 32), the half swap for partners 32 lanes away.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}
template <int M>  // the value of lane (lane ^ M), M = 8 or 16
__device__ __forceinline__ float swz_xor(float x) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x1F | (M << 10)));
}
// v + the value of lane (lane ^ 32), added in that order
__device__ __forceinline__ float add_xor32(float v) {
  float lo = v, hi = v;
  // lo's upper half <- hi's lower half: lo = the lower half's values in both
  // halves, hi = the upper half's
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
  return lo + hi;
}

// Maximum / sum within each half-wave of 32 lanes: pairs 1 and 2 apart
// (quad permutes), then each lane with its mirror in 8 and in 16 lanes (the
// partners hold equal values by then, so the mirror acts as a butterfly),
// then 16 apart.
__device__ __forceinline__ float half_maxf(float x) {
  x = fmaxf(x, dpp_mov<0xB1>(x));
  x = fmaxf(x, dpp_mov<0x4E>(x));
  x = fmaxf(x, dpp_mov<0x141>(x));
  x = fmaxf(x, dpp_mov<0x140>(x));
  return fmaxf(x, swz_xor<16>(x));
}
__device__ __forceinline__ float half_sumf(float x) {
  x += dpp_mov<0xB1>(x);
  x += dpp_mov<0x4E>(x);
  x += dpp_mov<0x141>(x);
  x += dpp_mov<0x140>(x);
  return x + swz_xor<16>(x);
}

// Orders a wave's LDS writes before its other lanes' reads (the LDS data
// of a workgroup of several waves is per wave, so no workgroup barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Waves of a workgroup that owns a whole (row, kv head, head group) and
// merges its parts in LDS: up to 8 (two per SIMD: the kernel needs ~240
// registers a wave, and 16 waves would leave it 128, spilling), with the
// partials (REP x D floats a wave) within 48 KB.
template <int D, int REP>
constexpr int fd_wg_waves() {
  constexpr int n = 49152 / (REP * D * 4);
  return n > 8 ? 8 : (n < 2 ? 2 : n);
}
// The shapes whose 8-wave workgroup fits its registers without spilling:
// bf16 / f16 (matrix-core scores) at 64 dims, or 128 dims and at most 4
// heads per group.
template <int DT, int D, int REP>
constexpr bool fd_wg_ok() {
  return DT != kF32 && (D == 64 || (D == 128 && REP <= 4));
}

// The in-launch merge of a (row, kv head, head group)'s parts
// (sdpa_vector.h:320-394), by the part that counted in last: the partials
// come back through device-coherent loads; all 64 lanes take D / 64 dims of
// a head each and issue every part's loads of the head together, one round
// trip per head.
template <int DT, int D, int REP>
__device__ __forceinline__ void fdecode_merge_rows(const AttnArgs& a, int64_t b, int h0, int nh,
                                                   int lane) {
  using E = Elem<DT>;
  constexpr int DPL = D / 64;  // dims per lane: 1, 2 or 4
  constexpr int kMaxP = 32;    // parts per round trip
  for (int r = 0; r < nh; r++) {
    const int h = h0 + r;
    const int64_t rh = b * a.Hq + h;
    const float* mlp = a.ws_ml + rh * a.n_parts * 2;
    const float* wo = a.ws_o + rh * a.n_parts * D + DPL * lane;
    float M = -3.402823466e38f, den = 0.0f, acc[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e++) acc[e] = 0.0f;
    for (int c = 0; c < a.n_parts; c += kMaxP) {
      float mj[kMaxP], lj[kMaxP], vj[kMaxP][DPL];
#pragma unroll
      for (int j = 0; j < kMaxP; j++) {
        const int pp = min(c + j, a.n_parts - 1);  // (clamped slots are selected away)
        const uint64_t w = __hip_atomic_load(reinterpret_cast<const uint64_t*>(mlp) + pp,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        mj[j] = __uint_as_float(static_cast<uint32_t>(w));
        lj[j] = __uint_as_float(static_cast<uint32_t>(w >> 32));
        const float* src = wo + static_cast<int64_t>(pp) * D;
        if constexpr (DPL == 1) {
          vj[j][0] = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
#pragma unroll
          for (int e = 0; e < DPL / 2; e++) {
            const uint64_t x = __hip_atomic_load(reinterpret_cast<const uint64_t*>(src) + e,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            vj[j][2 * e] = __uint_as_float(static_cast<uint32_t>(x));
            vj[j][2 * e + 1] = __uint_as_float(static_cast<uint32_t>(x >> 32));
          }
        }
      }
      float Mc = M;
#pragma unroll
      for (int j = 0; j < kMaxP; j++)
        if (c + j < a.n_parts) Mc = fmaxf(Mc, mj[j]);
      const float rsc = __expf(M - Mc);
      den *= rsc;
#pragma unroll
      for (int e = 0; e < DPL; e++) acc[e] *= rsc;
      M = Mc;
#pragma unroll
      for (int j = 0; j < kMaxP; j++) {
        if (c + j < a.n_parts) {
          const float w = __expf(mj[j] - M);
          den += w * lj[j];
#pragma unroll
          for (int e = 0; e < DPL; e++) acc[e] = fmaf(w, vj[j][e], acc[e]);
        }
      }
    }
    typename E::T* out = static_cast<typename E::T*>(a.out) + b * a.o_sb + h * a.o_sh + DPL * lane;
#pragma unroll
    for (int e = 0; e < DPL; e++) out[e] = E::from_f32(den > 0.0f ? acc[e] / den : 0.0f);
  }
}

template <int DT, int D, int REP, int NW = 1>
__global__ void __launch_bounds__(64 * NW) fdecode_kernel(AttnArgs a, int rep_total) {
  using E = Elem<DT>;
  constexpr int VEC = 16 / E::kBytes;  // elements per 16-byte load
  constexpr int KL = D / VEC;          // loads per key row
  constexpr int LPR = D / VEC;         // lanes per value row
  constexpr int RPI = 64 / LPR;        // value rows per load instruction
  static_assert(LPR <= 64 && 64 % LPR == 0, "value rows must tile a wave");
  static_assert(KL % 2 == 0 && kStep % RPI == 0, "key rows split in two halves, value rows tile a step");
  // bf16 / f16 K/V: the scores on matrix cores (S^T = K . Q^T, 16 tokens x
  // 16 columns of heads per MFMA, the raw queries as B operands, the scale
  // applied to the fp32 scores); f32 K/V: on the vector ALUs
  constexpr bool MF = DT != kF32;
  constexpr int KS = D / 32;  // 32-dim K steps of a key row
  static_assert(!MF || 2 * KS == KL / 2, "the key operands reuse the key-load registers");
  // (NW > 1: a workgroup of NW waves owns the whole row, wave w its part
  // w, and merges the parts in LDS at the end; each wave's LDS is its own)
  __shared__ float qs_g[NW][MF ? 1 : REP][MF ? 1 : D];
  __shared__ float ps_g[NW][REP][kStep];
  const int wv = NW > 1 ? static_cast<int>(threadIdx.x >> 6) : 0;
  float(*qs)[MF ? 1 : D] = qs_g[wv];
  float(*ps)[kStep] = ps_g[wv];
  auto step_sync = [&]() __attribute__((always_inline)) {
    if constexpr (NW > 1) wave_lds_sync();
    else __syncthreads();
  };

  const int lane = threadIdx.x & 63;
  const int part = static_cast<int>(blockIdx.x) * NW + wv;
  const int n_hg = (rep_total + REP - 1) / REP;
  const int hk = blockIdx.y / n_hg, hg = blockIdx.y % n_hg;
  const int64_t b = blockIdx.z;
  const int h0 = hk * rep_total + hg * REP;
  const int nh = min(REP, rep_total - hg * REP);
  const int64_t T = a.kv.T;
  const int64_t t_begin = static_cast<int64_t>(part) * a.part_tokens;
  const int64_t t_end = min<int64_t>(T, t_begin + a.part_tokens);

  const uint8_t* kbase = a.kv.kc.ptr + b * a.kv.kc.sb + hk * a.kv.kc.sh;
  const uint8_t* vbase = a.kv.vc.ptr + b * a.kv.vc.sb + hk * a.kv.vc.sh;
  const int64_t kst = a.kv.kc.st, vst = a.kv.vc.st;
  const int rs = lane / LPR, dg = lane % LPR;  // value phase: row slot, 16-byte run
  const int tok = lane & (kStep - 1), half = lane / kStep;
  // Loads of a step (t0): lanes tok and tok + 32 read half of key row
  // t0 + tok each; value row slot rs takes tokens t0 + rs, t0 + rs + RPI, ...
  // (rows past the end read the range's first row; their scores are masked
  // and their probabilities are 0).  All of a step's loads go out before
  // its first use, so a step waits for one memory round trip, not one per
  // group of loads; f32 at 256 dims would need more than 160 registers for
  // both sets, so there the value loads go out after the scores.  (Loading
  // the next step during this one's arithmetic keeps both sets live across
  // the loop: measured slower, fewer waves fit.)
  constexpr int NV = kStep / RPI;
  constexpr bool kVEarly = (KL / 2 + NV) * 4 <= 160;
  u32x4_t kw[KL / 2], vw[NV];
  // a cache update's deferred token: row new_t comes from its source rows,
  // and the range that holds it writes it into the cache (one head group)
  const int64_t new_t = a.has_new ? a.new_t : -1;
  const bool writes_new = new_t >= t_begin && new_t < t_end && hg == 0;
  const uint8_t* nkrow = a.has_new ? a.nk_ptr + b * a.nk_sb + hk * a.nk_sh : kbase;
  const uint8_t* nvrow = a.has_new ? a.nv_ptr + b * a.nv_sb + hk * a.nv_sh : vbase;
  // matrix-core layout: lane (mrow, kgrp) loads dims 32 s + 8 kgrp .. + 7 of
  // token t0 + 16 T + mrow into kw[T KS + s] (the A operand of step s, tile T)
  const int mrow = lane & 15, kgrp = lane >> 4;
  auto load_k = [&](int64_t t0) __attribute__((always_inline)) {
    if constexpr (MF) {
#pragma unroll
      for (int T = 0; T < 2; T++) {
        const int64_t tt = t0 + 16 * T + mrow;
        const int64_t t = tt < t_end ? tt : t_begin;
        const uint8_t* krow = (t == new_t ? nkrow : kbase + t * kst) + 16 * kgrp;
#pragma unroll
        for (int st = 0; st < KS; st++) kw[T * KS + st] = *(g_u32x4_t*)(krow + 64 * st);
      }
    } else {
      const int64_t t = t0 + tok < t_end ? t0 + tok : t_begin;
      const uint8_t* krow = (t == new_t ? nkrow : kbase + t * kst) + 16 * (KL / 2) * half;
#pragma unroll
      for (int c = 0; c < KL / 2; c++) kw[c] = *(g_u32x4_t*)(krow + 16 * c);
    }
  };
  auto load_v = [&](int64_t t0) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < NV; k++) {
      const int64_t tv = t0 + rs + RPI * k < t_end ? t0 + rs + RPI * k : t_begin;
      vw[k] = *(g_u32x4_t*)((tv == new_t ? nvrow : vbase + tv * vst) + 16 * dg);
    }
  };

  // the queries (times the scale) go to LDS; their loads go out first,
  // then the first step's key and value loads, so both latencies overlap
  constexpr int NQ = MF ? 1 : REP * D / 64;
  float qv[NQ];
  u32x4_t qb[MF ? KS : 1];  // matrix-core B operands: head mrow, dims 32 s + 8 kgrp .. + 7
  if constexpr (MF) {
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + b * a.q_sb +
                         static_cast<int64_t>(h0 + min(mrow, nh - 1)) * a.q_sh + 8 * kgrp;
#pragma unroll
    for (int st = 0; st < KS; st++) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t lo = qp[32 * st + 2 * e], hi = qp[32 * st + 2 * e + 1];
        qb[st][e] = mrow < nh ? (lo | (hi << 16)) : 0u;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < NQ; j++) {
      const int i = lane + 64 * j, r = i / D, d = i % D;
      qv[j] = r < nh ? E::load(static_cast<const typename E::T*>(a.q) + b * a.q_sb + (h0 + r) * a.q_sh + d)
                     : 0.0f;
    }
  }
  if (t_begin < t_end) {
    load_k(t_begin);
    if constexpr (kVEarly) load_v(t_begin);
  }
  if constexpr (!MF) {
#pragma unroll
    for (int j = 0; j < NQ; j++) {
      const int i = lane + 64 * j;
      qs[i / D][i % D] = qv[j] * a.scale;
    }
    step_sync();
  }
  float m[REP], l[REP], o[REP][VEC];
#pragma unroll
  for (int r = 0; r < REP; r++) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
    // an attention sink is one more logit with a zero value row, counted
    // once per row: the running max starts at it with sum 1
    // (sdpa_vector.h:93-96, :257-260)
    if (a.sinks && part == 0 && r < nh) {
      m[r] = load_as<DT>(a.sinks, a.sinks_dtype, h0 + r);
      l[r] = 1.0f;
    }
#pragma unroll
    for (int e = 0; e < VEC; e++) o[r][e] = 0.0f;
  }

  for (int64_t t0 = t_begin; t0 < t_end; t0 += kStep) {
    // ---- scores: lanes tok and tok + 32 own token t0 + tok, each half of
    // its dims
    const int64_t t = t0 + tok;
    const bool valid = t < t_end;
    if (t0 != t_begin) {
      load_k(t0);
      if constexpr (kVEarly) load_v(t0);
    }
    if constexpr (MF) {
      // ---- scores on matrix cores: lane (mrow, kgrp) ends with head mrow
      // of tokens t0 + 16 T + 4 kgrp + i
      f32x4_t acc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int st = 0; st < KS; st++)
#pragma unroll
        for (int T = 0; T < 2; T++) acc[T] = mfma16<DT>(kw[T * KS + st], qb[st], acc[T]);
      if constexpr (!kVEarly) load_v(t0);
      if (writes_new) {  // the new token's key row into the cache
#pragma unroll
        for (int T = 0; T < 2; T++) {
          if (t0 + 16 * T + mrow == new_t) {
            uint8_t* dst = const_cast<uint8_t*>(kbase) + new_t * kst + 16 * kgrp;
#pragma unroll
            for (int st = 0; st < KS; st++) *reinterpret_cast<u32x4_t*>(dst + 64 * st) = kw[T * KS + st];
          }
        }
      }
      float sc[2][4];
      float mx = -INFINITY;
#pragma unroll
      for (int T = 0; T < 2; T++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int64_t t = t0 + 16 * T + 4 * kgrp + i;
          float x = acc[T][i] * a.scale;
          bool vis = t < t_end && mrow < nh;
          if (vis && a.mask_mode >= 2) {
            const int64_t mo = b * a.m_sb + (h0 + mrow) * a.m_sh + t * a.m_st;
            if (a.mask_mode == 2) {
              vis = static_cast<const uint8_t*>(a.mask)[mo] != 0;
            } else {
              // the mask in the query dtype; keys below its lowest finite
              // value are skipped (sdpa_vector.h:105-121)
              const float add = load_as<DT>(a.mask, a.mask_dtype, mo);
              vis = add >= -E::kMax;
              x += add;
            }
          }
          sc[T][i] = vis ? x : -INFINITY;
          mx = fmaxf(mx, sc[T][i]);
        }
      // the step's max of head mrow over its four lanes, then the new
      // running max (this lane's head)
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      float m_own = m[0];
#pragma unroll
      for (int r = 1; r < REP; r++) m_own = mrow == r ? m[r] : m_own;
      const float mn_own = fmaxf(m_own, mx);
      float psum = 0.0f;
#pragma unroll
      for (int T = 0; T < 2; T++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float pr = (mn_own == -INFINITY || sc[T][i] == -INFINITY) ? 0.0f
                                                                         : __expf(sc[T][i] - mn_own);
          psum += pr;
          if (mrow < REP) ps[mrow][16 * T + 4 * kgrp + i] = pr;
        }
      psum += __shfl_xor(psum, 16);
      psum += __shfl_xor(psum, 32);
      // ---- online softmax per head (sdpa_vector.h:116-131): lane r holds
      // head r's new max and step sum
#pragma unroll
      for (int r = 0; r < REP; r++) {
        const float mn = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mn_own), r));
        const float ls = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, psum), r));
        float alpha = 1.0f;
        if (mn != -INFINITY) alpha = m[r] == -INFINITY ? 0.0f : __expf(m[r] - mn);
        l[r] = l[r] * alpha + ls;
        m[r] = mn;
#pragma unroll
        for (int e = 0; e < VEC; e++) o[r][e] *= alpha;
      }
    } else {
    float s[REP];
#pragma unroll
    for (int r = 0; r < REP; r++) s[r] = 0.0f;
#pragma unroll
    for (int c = 0; c < KL / 2; c++) {
      float kv[VEC];
      unpack16<DT>(kw[c], kv);
      const int q0 = VEC * (c + (KL / 2) * half);
#pragma unroll
      for (int r = 0; r < REP; r++)
#pragma unroll
        for (int e = 0; e < VEC; e++) s[r] = fmaf(qs[r][q0 + e], kv[e], s[r]);
    }
    if constexpr (!kVEarly) load_v(t0);
    if (writes_new && t == new_t) {  // the new token's key row into the cache
      uint8_t* dst = const_cast<uint8_t*>(kbase) + new_t * kst + 16 * (KL / 2) * half;
#pragma unroll
      for (int c = 0; c < KL / 2; c++) *reinterpret_cast<u32x4_t*>(dst + 16 * c) = kw[c];
    }

#pragma unroll
    for (int r = 0; r < REP; r++) s[r] = add_xor32(s[r]);
#pragma unroll
    for (int r = 0; r < REP; r++) {
      bool vis = valid && r < nh;
      if (vis && a.mask_mode >= 2) {
        const int64_t mo = b * a.m_sb + (h0 + r) * a.m_sh + t * a.m_st;
        if (a.mask_mode == 2) {
          vis = static_cast<const uint8_t*>(a.mask)[mo] != 0;
        } else {
          // the mask in the query dtype; keys below its lowest finite
          // value are skipped (sdpa_vector.h:105-121)
          const float add = load_as<DT>(a.mask, a.mask_dtype, mo);
          vis = add >= -E::kMax;
          s[r] += add;
        }
      }
      s[r] = vis ? s[r] : -INFINITY;
    }
    // ---- online softmax per head (sdpa_vector.h:116-131)
#pragma unroll
    for (int r = 0; r < REP; r++) {
      const float mn = fmaxf(m[r], half_maxf(s[r]));
      float p = 0.0f, alpha = 1.0f;
      if (mn != -INFINITY) {
        p = s[r] == -INFINITY ? 0.0f : __expf(s[r] - mn);
        alpha = m[r] == -INFINITY ? 0.0f : __expf(m[r] - mn);
      }
      l[r] = l[r] * alpha + half_sumf(p);
      m[r] = mn;
      if (half == 0) ps[r][tok] = p;
#pragma unroll
      for (int e = 0; e < VEC; e++) o[r][e] *= alpha;
    }
    }
    step_sync();
#pragma unroll
    for (int k = 0; k < NV; k++) {
      const int tt = rs + RPI * k;
      if (writes_new && t0 + tt == new_t)  // the new token's value row into the cache
        *reinterpret_cast<u32x4_t*>(const_cast<uint8_t*>(vbase) + new_t * vst + 16 * dg) = vw[k];
      float vv[VEC];
      unpack16<DT>(vw[k], vv);
#pragma unroll
      for (int r = 0; r < REP; r++) {
        const float p = ps[r][tt];
#pragma unroll
        for (int e = 0; e < VEC; e++) o[r][e] = fmaf(p, vv[e], o[r][e]);
      }
    }
    step_sync();
  }

  // the row slots of a run hold disjoint tokens: sum them
#pragma unroll
  for (int r = 0; r < REP; r++)
#pragma unroll
    for (int e = 0; e < VEC; e++) {
      if constexpr (LPR <= 8) o[r][e] += swz_xor<8>(o[r][e]);
      if constexpr (LPR <= 16) o[r][e] += swz_xor<16>(o[r][e]);
      if constexpr (LPR <= 32) o[r][e] = add_xor32(o[r][e]);
    }
  if constexpr (NW > 1) {
    // ---- the workgroup's parts merge in LDS (sdpa_vector.h:320-394): each
    // wave's (o, max, sum) per head, then every thread one (head, dim)
    __shared__ float mo_g[NW][REP][D];
    __shared__ float ml_g[NW][REP][2];
    if (rs == 0) {
#pragma unroll
      for (int r = 0; r < REP; r++) {
#pragma unroll
        for (int e = 0; e < VEC; e++) mo_g[wv][r][VEC * dg + e] = o[r][e];
        if (dg == 0) {
          ml_g[wv][r][0] = m[r];
          ml_g[wv][r][1] = l[r];
        }
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < nh * D; idx += 64 * NW) {
      const int r = idx / D, d = idx % D;
      float M = -3.402823466e38f;
#pragma unroll
      for (int w = 0; w < NW; w++) M = fmaxf(M, ml_g[w][r][0]);
      float den = 0.0f, acc = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; w++) {
        const float f = __expf(ml_g[w][r][0] - M);
        den = fmaf(f, ml_g[w][r][1], den);
        acc = fmaf(f, mo_g[w][r][d], acc);
      }
      typename E::T* out = static_cast<typename E::T*>(a.out) + b * a.o_sb + (h0 + r) * a.o_sh + d;
      *out = E::from_f32(den > 0.0f ? acc / den : 0.0f);
    }
    return;
  }
  const bool merge_here = a.n_parts > 1 && a.counters;
  if (rs == 0) {
#pragma unroll
    for (int r = 0; r < REP; r++) {
      if (r >= nh) break;
      const int h = h0 + r;
      const int d0 = VEC * dg;
      if (a.n_parts == 1) {
        const float inv = l[r] > 0.0f ? 1.0f / l[r] : 0.0f;
        typename E::T* out = static_cast<typename E::T*>(a.out) + b * a.o_sb + h * a.o_sh + d0;
#pragma unroll
        for (int e = 0; e < VEC; e++) out[e] = E::from_f32(o[r][e] * inv);
      } else if (merge_here) {
        const int64_t base = (b * a.Hq + h) * a.n_parts + part;
        uint64_t* wo = reinterpret_cast<uint64_t*>(a.ws_o + base * D + d0);
#pragma unroll
        for (int e = 0; e < VEC / 2; e++)
          __hip_atomic_store(wo + e, pack_f2(o[r][2 * e], o[r][2 * e + 1]), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        if (dg == 0)
          __hip_atomic_store(reinterpret_cast<uint64_t*>(a.ws_ml + base * 2), pack_f2(m[r], l[r]),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        const int64_t base = (b * a.Hq + h) * a.n_parts + part;
        float* wo = a.ws_o + base * D + d0;
#pragma unroll
        for (int e = 0; e < VEC; e++) wo[e] = o[r][e];
        if (dg == 0) {
          a.ws_ml[base * 2] = m[r];
          a.ws_ml[base * 2 + 1] = l[r];
        }
      }
    }
  }
  if (!merge_here) return;
  // this part's partial stores are complete before it counts itself in
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  uint32_t* cnt = a.counters + (b * a.Hkv + hk) * n_hg + hg;
  uint32_t before = 0;
  if (lane == 0) before = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  before = __builtin_amdgcn_readfirstlane(before);
  if (before != static_cast<uint32_t>(a.n_parts - 1)) return;
  // the last part merges every part of the group's heads, then zeroes the
  // counter for the next launch
  if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  fdecode_merge_rows<DT, D, REP>(a, b, h0, nh, lane);
}

template <int DT, int D, int R>
void launch_r(const AttnArgs& a, int64_t rows, int rep, int n_hg, hipStream_t st) {
  const TimedLaunch tl = timing_prepare(kTimeFDecode);
  if (a.wg_parts > 0) {
    // one workgroup per (row, kv head, head group), its parts merged in LDS
    if constexpr (fd_wg_ok<DT, D, R>()) {
      constexpr int NW = fd_wg_waves<D, R>();
      VKV_CHECK(a.wg_parts <= NW && a.n_parts == a.wg_parts, "workgroup parts");
      const dim3 grid(1, a.Hkv * n_hg, static_cast<unsigned>(rows));
      hipExtLaunchKernelGGL((fdecode_kernel<DT, D, R, NW>), grid, dim3(64 * NW), 0, st, tl.start,
                            tl.stop, 0, a, rep);
    } else {
      throw Error("no workgroup float decode for this shape");
    }
  } else {
    const dim3 grid(a.n_parts, a.Hkv * n_hg, static_cast<unsigned>(rows));
    hipExtLaunchKernelGGL((fdecode_kernel<DT, D, R>), grid, dim3(64), 0, st, tl.start, tl.stop, 0,
                          a, rep);
  }
  VKV_HIP(hipGetLastError());
  timing_commit(tl);
}

// Query heads a wave takes (its head group): all of a kv head's, up to 8,
// so that each key row is read once for them.  The workgroup form of a
// launch of at most 512 (row, query head)s takes one head a workgroup: the
// launch then has 4-8x the workgroups, each reading its K/V from L2 (config
// 1, one row of 8 kv heads x 4: kernel 13.0 us at four heads, 10.2 at one).
int fd_group_heads(int64_t rows, int Hkv, int rep, bool wg) {
  if (wg && rows * Hkv * rep <= 512) return 1;
  return rep <= 1 ? 1 : rep <= 2 ? 2 : rep <= 4 ? 4 : 8;
}

template <int DT, int D>
void launch_d(const AttnArgs& a, int64_t rows, hipStream_t st) {
  const int rep = a.Hq / a.Hkv;
  const int R = fd_group_heads(rows, a.Hkv, rep, a.wg_parts > 0);
  const int n_hg = (rep + R - 1) / R;
  if (R == 1) launch_r<DT, D, 1>(a, rows, rep, n_hg, st);
  else if (R == 2) launch_r<DT, D, 2>(a, rows, rep, n_hg, st);
  else if (R == 4) launch_r<DT, D, 4>(a, rows, rep, n_hg, st);
  else launch_r<DT, D, 8>(a, rows, rep, n_hg, st);
}

template <int DT>
void launch_dt(const AttnArgs& a, int64_t rows, hipStream_t st) {
  if (a.D == 64) launch_d<DT, 64>(a, rows, st);
  else if (a.D == 128) launch_d<DT, 128>(a, rows, st);
  else launch_d<DT, 256>(a, rows, st);
}

}  // namespace

bool fdecode_supported(int dtype, int bits, bool qsem, const AttnArgs& a) {
  if (bits != 0 || qsem || a.L != 1 || a.kv.table || a.kv.qfmt || a.kv.seq_lens) return false;
  if (a.D != a.Dv || (a.D != 64 && a.D != 128 && a.D != 256)) return false;
  if (a.Hq % a.Hkv) return false;
  if (a.mask_mode < 0 || a.mask_mode > 3) return false;
  // f32 rows at 128 dims with more than 4 query heads a kv head, or at 256
  // dims with more than 2, need more registers than a wave has (the step's
  // f32 key and value rows beside the group's accumulators): those variants
  // spill hundreds of registers to scratch and ran 1.9-4.7x slower than the
  // generic kernel, which therefore takes them
  const int rep = a.Hq / a.Hkv;
  if (dtype == kF32 && ((a.D == 128 && rep > 4) || (a.D == 256 && rep > 2))) return false;
  const int es = elem_bytes(dtype);
  // 16-byte loads of key and value rows
  auto al = [](const void* p, int64_t s0, int64_t s1, int64_t s2) {
    return reinterpret_cast<uintptr_t>(p) % 16 == 0 && s0 % 16 == 0 && s1 % 16 == 0 && s2 % 16 == 0;
  };
  (void)es;
  return al(a.kv.kc.ptr, a.kv.kc.sb, a.kv.kc.sh, a.kv.kc.st) &&
         al(a.kv.vc.ptr, a.kv.vc.sb, a.kv.vc.sh, a.kv.vc.st);
}

int fdecode_parts(int64_t rows_x_heads, int64_t T, int32_t* part_tokens, int waves) {
  // about `waves` (default 2048) waves, kStep-token steps
  if (waves <= 0) waves = 2048;
  int64_t parts = std::max<int64_t>(1, waves / std::max<int64_t>(1, rows_x_heads));
  parts = std::min<int64_t>(parts, std::max<int64_t>(1, (T + kStep - 1) / kStep));
  int64_t pt = (T + parts - 1) / parts;
  pt = std::max<int64_t>(kStep, (pt + kStep - 1) / kStep * kStep);
  *part_tokens = static_cast<int32_t>(pt);
  return static_cast<int>(std::max<int64_t>(1, (T + pt - 1) / pt));
}

int fdecode_wg_parts(int64_t rows, int Hq, int Hkv, int64_t T, int D, int dtype,
                     int32_t* part_tokens) {
  // launches of at most kWgBytes of K/V: few (row, head group)s whose parts
  // the global merge would cost more than they save
  constexpr int64_t kWgBytes = int64_t{8} << 20;
  if (rows * Hkv * T * D * 2 * elem_bytes(dtype) > kWgBytes) return 0;
  const int R = fd_group_heads(rows, Hkv, Hq / Hkv, true);
  if (dtype == kF32 || !(D == 64 || (D == 128 && R <= 4))) return 0;  // fd_wg_ok
  int nw = 8;
  switch (D * 8 + R) {  // fd_wg_waves<D, R>()
#define VKV_WG(DD, RR) case DD * 8 + RR: nw = fd_wg_waves<DD, RR>(); break;
    VKV_WG(64, 1) VKV_WG(64, 2) VKV_WG(64, 4) VKV_WG(64, 8)
    VKV_WG(128, 1) VKV_WG(128, 2) VKV_WG(128, 4)
#undef VKV_WG
    default: return 0;
  }
  const int64_t steps = std::max<int64_t>(1, (T + kStep - 1) / kStep);
  const int64_t parts = std::min<int64_t>(nw, steps);
  const int64_t pt = (steps + parts - 1) / parts * kStep;
  *part_tokens = static_cast<int32_t>(pt);
  return static_cast<int>((std::max<int64_t>(T, 1) + pt - 1) / pt);
}

void launch_fdecode(int dtype, const AttnArgs& a, int64_t rows, hipStream_t st) {
  if (rows <= 0) return;
  // a causal mask leaves one query token every key
  AttnArgs b = a;
  if (b.mask_mode == 1) b.mask_mode = 0;
  switch (dtype) {
    case kF32: launch_dt<kF32>(b, rows, st); break;
    case kF16: launch_dt<kF16>(b, rows, st); break;
    case kBF16: launch_dt<kBF16>(b, rows, st); break;
    default: throw Error("unsupported dtype");
  }
  if (b.n_parts > 1 && !b.counters && b.wg_parts == 0) launch_attn_combine(dtype, b, rows, st);
}

static int fdecode_heads_per_group(int Hq, int Hkv) {
  const int rep = Hq / Hkv;
  return rep <= 1 ? 1 : rep <= 2 ? 2 : rep <= 4 ? 4 : 8;
}

int fdecode_counter_count(int Hq, int Hkv) {
  const int rep = Hq / Hkv, R = fdecode_heads_per_group(Hq, Hkv);
  return Hkv * ((rep + R - 1) / R);
}

bool fdecode_merge_here(int n_parts, int Dv, int Hq, int Hkv) {
  // partial floats the last part of a head group reads back
  constexpr int64_t kMaxMergeFloats = 12288;
  return static_cast<int64_t>(n_parts) * Dv * fdecode_heads_per_group(Hq, Hkv) <= kMaxMergeFloats;
}

}  // namespace vkv
