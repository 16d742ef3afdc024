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
//   * scores: lanes t and t + 32 own token t, each taking half of its key
//     row with 16-byte loads (every byte of a row used), against the
//     queries of the group's REP heads in LDS; one lane swap adds the
//     halves.  Two lanes per token give a launch twice the waves of one
//     lane per token for the same bytes (a 33.6 MB D = 256 decode: 14.9 ->
//     12.3 us).
//   * online softmax per head over the 32 scores (DPP reductions within
//     each half-wave), the probabilities into LDS;
//   * values: lanes own 16-byte runs of a value row, D/8 (bf16/f16) or D/4
//     (f32) lanes per row, so every load instruction reads whole rows;
//     the lanes that share a run sum their tokens at the end.
// No matrix cores: at REP <= 8 query heads per kv head the contraction is
// ~1 FMA per KV byte, well under the vector ALUs' rate, so the kernel runs
// at the memory's pace.
#include <algorithm>

#include "vkv_device.h"
#include <hip/hip_ext.h>
#include "vkv_internal.h"

namespace vkv {

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;

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

// Maximum / sum within each half-wave of 32 lanes.
__device__ __forceinline__ float half_maxf(float x) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float half_sumf(float x) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

template <int DT, int D, int REP>
__global__ void __launch_bounds__(64) fdecode_kernel(AttnArgs a, int rep_total) {
  using E = Elem<DT>;
  constexpr int VEC = 16 / E::kBytes;  // elements per 16-byte load
  constexpr int KL = D / VEC;          // loads per key row
  constexpr int LPR = D / VEC;         // lanes per value row
  constexpr int RPI = 64 / LPR;        // value rows per load instruction
  static_assert(LPR <= 64 && 64 % LPR == 0, "value rows must tile a wave");
  static_assert(KL % 2 == 0 && kStep % RPI == 0, "key rows split in two halves, value rows tile a step");
  __shared__ float qs[REP][D];
  __shared__ float ps[REP][kStep];

  const int lane = threadIdx.x;
  const int part = blockIdx.x;
  const int n_hg = (rep_total + REP - 1) / REP;
  const int hk = blockIdx.y / n_hg, hg = blockIdx.y % n_hg;
  const int64_t b = blockIdx.z;
  const int h0 = hk * rep_total + hg * REP;
  const int nh = min(REP, rep_total - hg * REP);
  const int64_t T = a.kv.T;
  const int64_t t_begin = static_cast<int64_t>(part) * a.part_tokens;
  const int64_t t_end = min<int64_t>(T, t_begin + a.part_tokens);

  for (int i = lane; i < REP * D; i += 64) {
    const int r = i / D, d = i % D;
    float qv = 0.0f;
    if (r < nh)
      qv = E::load(static_cast<const typename E::T*>(a.q) + b * a.q_sb + (h0 + r) * a.q_sh + d) *
           a.scale;
    qs[r][d] = qv;
  }
  __syncthreads();

  const uint8_t* kbase = a.kv.kc.ptr + b * a.kv.kc.sb + hk * a.kv.kc.sh;
  const uint8_t* vbase = a.kv.vc.ptr + b * a.kv.vc.sb + hk * a.kv.vc.sh;
  const int64_t kst = a.kv.kc.st, vst = a.kv.vc.st;
  const int rs = lane / LPR, dg = lane % LPR;  // value phase: row slot, 16-byte run

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

  const int tok = lane & (kStep - 1), half = lane / kStep;
  for (int64_t t0 = t_begin; t0 < t_end; t0 += kStep) {
    // ---- scores: lanes tok and tok + 32 own token t0 + tok, each half of
    // its dims (rows past the end read the range's first row and are masked)
    const int64_t t = t0 + tok;
    const bool valid = t < t_end;
    const uint8_t* krow = kbase + (valid ? t : t_begin) * kst + 16 * (KL / 2) * half;
    float s[REP];
#pragma unroll
    for (int r = 0; r < REP; r++) s[r] = 0.0f;
#pragma unroll 4
    for (int c = 0; c < KL / 2; c++) {
      const u32x4_t w = *(g_u32x4_t*)(krow + 16 * c);
      float kv[VEC];
      unpack16<DT>(w, kv);
      const int q0 = VEC * (c + (KL / 2) * half);
#pragma unroll
      for (int r = 0; r < REP; r++)
#pragma unroll
        for (int e = 0; e < VEC; e++) s[r] = fmaf(qs[r][q0 + e], kv[e], s[r]);
    }
#pragma unroll
    for (int r = 0; r < REP; r++) s[r] += __shfl_xor(s[r], kStep);
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
    __syncthreads();
    // ---- values: row slot rs takes tokens t0 + rs, t0 + rs + RPI, ...
    // (probability 0 past the end, where the row read is clamped)
#pragma unroll 4
    for (int k = 0; k < kStep / RPI; k++) {
      const int tt = rs + RPI * k;
      const int64_t tv = t0 + tt;
      const uint8_t* vrow = vbase + (tv < t_end ? tv : t_begin) * vst + 16 * dg;
      const u32x4_t w = *(g_u32x4_t*)(vrow);
      float vv[VEC];
      unpack16<DT>(w, vv);
#pragma unroll
      for (int r = 0; r < REP; r++) {
        const float p = ps[r][tt];
#pragma unroll
        for (int e = 0; e < VEC; e++) o[r][e] = fmaf(p, vv[e], o[r][e]);
      }
    }
    __syncthreads();
  }

  // the row slots of a run hold disjoint tokens: sum them
#pragma unroll
  for (int r = 0; r < REP; r++)
#pragma unroll
    for (int e = 0; e < VEC; e++)
#pragma unroll
      for (int off = LPR; off < 64; off <<= 1) o[r][e] += __shfl_xor(o[r][e], off);
  if (rs != 0) return;
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

template <int DT, int D>
void launch_d(const AttnArgs& a, int64_t rows, hipStream_t st) {
  const int rep = a.Hq / a.Hkv;
  const int R = rep <= 1 ? 1 : rep <= 2 ? 2 : rep <= 4 ? 4 : 8;
  const int n_hg = (rep + R - 1) / R;
  const dim3 grid(a.n_parts, a.Hkv * n_hg, static_cast<unsigned>(rows));
  const TimedLaunch tl = timing_prepare(kTimeFDecode);
  if (R == 1)
    hipExtLaunchKernelGGL((fdecode_kernel<DT, D, 1>), grid, dim3(64), 0, st, tl.start, tl.stop, 0, a, rep);
  else if (R == 2)
    hipExtLaunchKernelGGL((fdecode_kernel<DT, D, 2>), grid, dim3(64), 0, st, tl.start, tl.stop, 0, a, rep);
  else if (R == 4)
    hipExtLaunchKernelGGL((fdecode_kernel<DT, D, 4>), grid, dim3(64), 0, st, tl.start, tl.stop, 0, a, rep);
  else
    hipExtLaunchKernelGGL((fdecode_kernel<DT, D, 8>), grid, dim3(64), 0, st, tl.start, tl.stop, 0, a, rep);
  VKV_HIP(hipGetLastError());
  timing_commit(tl);
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
  if (b.n_parts > 1) launch_attn_combine(dtype, b, rows, st);
}

}  // namespace vkv
