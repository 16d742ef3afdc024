// vkv_decode.hip -- decode attention over paged affine (4/8-bit) bf16 KV on
// gfx950 matrix cores.
//
// Semantics: quantizedScaledDotProductAttention
// (Libraries/MLXLMCommon/KVCache.swift:1909-1997) for one query token per
// sequence: queries scaled in bf16, scores q.dequant(K) accumulated in fp32
// and stored in bf16 as the reference's quantizedMM stores them, softmax,
// P.dequant(V), fp32 accumulation, output rounded to bf16.  Split-K partials are merged as
// sdpa_vector_2pass_2 merges them
// (Source/Cmlx/mlx-generated/metal/sdpa_vector.h:320-394).
//
// Arithmetic.  Both contractions run as 16x16x32 bf16 MFMAs directly on the
// codes, so the vector ALUs only unpack codes and run the softmax:
//   * a 4-bit value code c enters as bf16(128 + c), bit pattern 0x4300 | c,
//     which is exact; an 8-bit value code c = 16*hi + lo enters as two
//     operands, bf16(128 + lo) = 0x4300 | lo and bf16(2048 + 16*hi) =
//     0x4500 | hi, whose sum is c + 2176 (MAG); key codes use smaller
//     offsets (KMAG = 16 + c, or 272 + c as bf16(16 + lo) + bf16(256 + 16 hi)),
//     which keeps the fp32 score error small before its rounding to bf16;
//   * per-(token, group) scale s and bias b are applied around the
//     contraction:  q.(s*c + b) = s * q.(KMAG + c) + (b - KMAG s) * sum(q), and
//     sum_t p_t (s_t c_t + b_t) = sum_t P_t (MAG + c_t)
//                                 + sum_t p_t (b_t + C0 s_t) - (MAG + C0) sum_t P_t
//     with P_t = p_t s_t carried as two bf16 operands (hi + lo, about 16
//     significant bits between them; a single bf16 P would put a 2^-9
//     relative error on the code part s*c).  The offset sum uses the same
//     hi + lo values the MFMA consumed, so it cancels to fp32 rounding, and
//     the centre C0 (the code midpoint) leaves a residual error of the size
//     of the value's own deviation from its group midpoint.
//
// Work layout.  A 64-token step of one (sequence, kv head) is one pass.  The
// score MFMA is block diagonal: with HP query heads per part (HP = 4 for up
// to 4 query heads per kv head, else 8; more than 8 are split into head
// groups of 8 on separate workgroups) the 16 output columns are PP = 16 / HP
// parts x HP heads, and the 32-element K dimension is split between the parts, so one
// 16x16 output tile carries 16 * PP tokens x HP heads and every lane holds 4
// live scores.  Lane l = n + 16 lg (n = column) sees tokens
// 32 s + 8 lg + off(q, i) of head n % HP, where (s, q) enumerate the parts of
// the step and off() is the order in which the value operand's K dimension
// visits the 8 tokens of a value word.  The probabilities of head h then
// reach the P.V operand of lane h + 16 lg by DPP row rotations (no LDS), and
// the P.V output holds value dim 16 t + 4 lg + i of head n in lane n + 16 lg.
// The running max is refreshed lazily (only when a score exceeds it by more
// than kTau), which needs no cross-lane reduction on the common path and
// bounds probabilities by e^kTau.
//
// Work split.  The (sequence, kv head, head group, 64-token step) units of
// the whole batch are laid end to end, each (sequence, head group) pair led
// by kSegCost extra cost units for its finalize, and every wave takes an
// equal contiguous range of cost units, so mixed sequence lengths cost no
// load imbalance.  A range crosses a few (sequence, head) segments; at each
// boundary the wave finalizes the segment (the output itself when the
// segment covers the whole sequence, else an (o, max, sum) partial, merged
// as sdpa_vector_2pass_2 merges) and rebuilds its wave-local query table.
// The next unit's KV loads are in flight while the current unit computes,
// and the next segment's queries while the current segment does.  Up to 128
// dims a workgroup is the 8 waves of one CU (two per SIMD), and the two
// waves of a SIMD trade instruction-issue priority so that neither finishes
// long before the other.
//
// Merge.  Where the host passes counters, the partials merge inside the
// launch: a wave stores its partials with agent-coherent stores and counts
// them in on per-pair counters only at its range's end (a count right after
// the stores would wait for every prefetch in flight), and the wave that
// counts a pair's last partial merges it (device-scope fences instead of
// coherent stores would write back and invalidate the XCD's L2 per
// partial).  Otherwise qdecode_combine_kernel merges, in a launch of its
// own, through the same merge step.
#include <algorithm>
#include <mutex>
#include <string>
#include <utility>

#include "vkv_device.h"
#include <hip/hip_ext.h>

#include "vkv_internal.h"

namespace vkv {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
// global-memory views: KV loads must not become flat loads, which would
// also count against the LDS wait counter
typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;
typedef __attribute__((address_space(1))) const u32x2_t g_u32x2_t;
typedef __attribute__((address_space(1))) const uint32_t g_u32_t;

constexpr float kTau = 8.0f;
constexpr float kLog2e = 1.4426950408889634f;

// 2^x with the hardware v_exp_f32 (results below 2^-126 flush to zero,
// which is immaterial for softmax weights; exp2f adds a denormal-safe
// rescaling around it).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
constexpr int kMaxRange = 64;   // units (64-token steps) per wave, at most
constexpr int kMaxSeqs = 256;   // sequences per launch (the host splits larger batches)
constexpr int kMaxParts = 32;   // partials per (sequence, head pair), at most, up to
                                // kMaxRange * (kMaxParts - 1) * 64 tokens; longer
                                // sequences raise the launch's limit (max_parts)
// Work-split cost of a (sequence, head pair) beyond its 64-token steps: the
// finalize and set-up at a segment boundary take about as long as a step
// (0.7 steps measured at 128 dims, 4 bits), so the ranges count each pair
// as steps + kSegCost units and a range that crosses many short sequences
// gets fewer steps.
constexpr int kSegCost = 1;

template <int... Is, class F>
__device__ __forceinline__ void sfor_impl(std::integer_sequence<int, Is...>, F&& f) {
  (f(std::integral_constant<int, Is>{}), ...);
}
// Compile-time loop: f(std::integral_constant<int, I>) for I in [0, N).
template <int N, class F>
__device__ __forceinline__ void sfor(F&& f) {
  sfor_impl(std::make_integer_sequence<int, N>{}, f);
}

__device__ __forceinline__ f32x4_t mfma(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
// The score contraction in the cache's dtype: bf16 operands, or f16 ones for
// an f16 cache (its queries keep their 11 bits).  The value contraction is
// bf16 for both.
template <int DT>
__device__ __forceinline__ f32x4_t mfma_qk(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  if constexpr (DT == kF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  else
    return mfma(a, b, c);
}

// The bf16 exponent patterns OR-ed onto the codes, held in VGPRs the
// compiler cannot see through: with both the mask and the pattern as
// literals it emits v_and + v_or, with the pattern in a register one
// v_and_or_b32.
struct Magic {
  uint32_t m128, m2048;  // 0x43004300 (128 + c), 0x45004500 (2048 + 16 c)
  uint32_t m16, m256;    // 0x41804180 (16 + c), 0x43804380 (256 + 16 c)
  __device__ __forceinline__ Magic()
      : m128(0x43004300u), m2048(0x45004500u), m16(0x41804180u), m256(0x43804380u) {
    asm volatile("" : "+v"(m128), "+v"(m2048), "+v"(m16), "+v"(m256));
  }
};

// 8 nibbles -> 8 bf16 (128 + nibble); register r holds nibbles (r, r + 4).
__device__ __forceinline__ u32x4_t nib_magic(uint32_t w, const Magic& mg) {
  u32x4_t r;
  r[0] = (w & 0x000F000Fu) | mg.m128;
  r[1] = ((w >> 4) & 0x000F000Fu) | mg.m128;
  r[2] = ((w >> 8) & 0x000F000Fu) | mg.m128;
  r[3] = ((w >> 12) & 0x000F000Fu) | mg.m128;
  return r;
}

// Key operands with small offsets: 8 nibbles -> bf16 (16 + nibble), whose
// mantissa unit is 1/8, so the nibble goes in three bits up.  The score is
// s * q.(KMAG + c) + (b - KMAG s) * sum(q); the fp32 rounding of the two
// KMAG terms that cancel grows with KMAG, and the scores are rounded to
// bf16 afterwards, so a small KMAG keeps them on the same side of a bf16
// rounding boundary as the exact score far more often (16 against 128: ~4x
// fewer flips on outlier data).
__device__ __forceinline__ u32x4_t nib_magic_k(uint32_t w, const Magic& mg) {
  u32x4_t r;
  r[0] = ((w << 3) & 0x00780078u) | mg.m16;
  r[1] = ((w >> 1) & 0x00780078u) | mg.m16;
  r[2] = ((w >> 5) & 0x00780078u) | mg.m16;
  r[3] = ((w >> 9) & 0x00780078u) | mg.m16;
  return r;
}

// 8 bytes (x then y) -> low nibbles as bf16 (128 + lo) and high nibbles as
// bf16 (2048 + 16 hi); register order (b0, b2), (b1, b3) of x, then of y.
__device__ __forceinline__ void byte_magic(uint32_t x, uint32_t y, const Magic& mg, u32x4_t& lo,
                                           u32x4_t& hi) {
  lo[0] = (x & 0x000F000Fu) | mg.m128;
  lo[1] = ((x >> 8) & 0x000F000Fu) | mg.m128;
  lo[2] = (y & 0x000F000Fu) | mg.m128;
  lo[3] = ((y >> 8) & 0x000F000Fu) | mg.m128;
  hi[0] = ((x >> 4) & 0x000F000Fu) | mg.m2048;
  hi[1] = ((x >> 12) & 0x000F000Fu) | mg.m2048;
  hi[2] = ((y >> 4) & 0x000F000Fu) | mg.m2048;
  hi[3] = ((y >> 12) & 0x000F000Fu) | mg.m2048;
}

// f16 key operands (an f16 cache): 8 nibbles -> f16 (16 + nibble), whose
// mantissa unit is 1/64 (the nibble six bits up), KMAG = 16; 8 bytes ->
// f16 (256 + byte), unit 1/4, KMAG = 256, one operand per 8 dims (bytes
// (b0, b2), (b1, b3) of x, then of y, the order of byte_magic_k's lo).
__device__ __forceinline__ u32x4_t nib_magic_k16(uint32_t w) {
  uint32_t m = 0x4C004C00u;
  asm volatile("" : "+v"(m));
  u32x4_t r;
  r[0] = ((w << 6) & 0x03C003C0u) | m;
  r[1] = ((w << 2) & 0x03C003C0u) | m;
  r[2] = ((w >> 2) & 0x03C003C0u) | m;
  r[3] = ((w >> 6) & 0x03C003C0u) | m;
  return r;
}
__device__ __forceinline__ u32x4_t byte_magic_k16(uint32_t x, uint32_t y) {
  uint32_t m = 0x5C005C00u;
  asm volatile("" : "+v"(m));
  u32x4_t r;
  r[0] = ((x << 2) & 0x03FC03FCu) | m;
  r[1] = ((x >> 6) & 0x03FC03FCu) | m;
  r[2] = ((y << 2) & 0x03FC03FCu) | m;
  r[3] = ((y >> 6) & 0x03FC03FCu) | m;
  return r;
}

// The same for key operands with small offsets: low nibbles as bf16
// (16 + lo), high nibbles as bf16 (256 + 16 hi), KMAG = 272.
__device__ __forceinline__ void byte_magic_k(uint32_t x, uint32_t y, const Magic& mg, u32x4_t& lo,
                                             u32x4_t& hi) {
  lo[0] = ((x << 3) & 0x00780078u) | mg.m16;
  lo[1] = ((x >> 5) & 0x00780078u) | mg.m16;
  lo[2] = ((y << 3) & 0x00780078u) | mg.m16;
  lo[3] = ((y >> 5) & 0x00780078u) | mg.m16;
  hi[0] = ((x >> 1) & 0x00780078u) | mg.m256;
  hi[1] = ((x >> 9) & 0x00780078u) | mg.m256;
  hi[2] = ((y >> 1) & 0x00780078u) | mg.m256;
  hi[3] = ((y >> 9) & 0x00780078u) | mg.m256;
}

// Dim (within an 8-dim unit) carried by MFMA K element j of a key operand:
// 4-bit registers pair nibbles (p, p + 4), 8-bit pair bytes (0, 2), (1, 3).
template <int BITS>
__device__ __forceinline__ int kslot(int j) {
  if constexpr (BITS == 4) return (j & 1) ? (j >> 1) + 4 : (j >> 1);
  const int r = j & 3;
  return (j & 4) | (r == 1 ? 2 : r == 2 ? 1 : r);
}

// Token (within the 8 tokens of a value word) of score register i of a lane
// whose part is q: the pairs (i0, i1) and (i2, i3) are exactly the token
// pairs one value-operand register holds, so a lane packs its own pairs.
template <int BITS>
__device__ __forceinline__ int tok_off(int q, int i) {
  if constexpr (BITS == 4) return 2 * q + (i >> 1) + 4 * (i & 1);
  return 4 * q + 2 * (i & 1) + (i >> 1);
}

// Value of lane (lane + K) within this lane's row of 16 (DPP row_ror:N
// reads lane (i - N) mod 16).
template <int K>
__device__ __forceinline__ uint32_t row_read(uint32_t x) {
  if constexpr (K == 0) {
    return x;
  } else {
    // mov_dpp has no "old" operand (all lanes are written), so the compiler
    // does not materialize one first
    return __builtin_amdgcn_mov_dpp(x, 0x120 + (16 - K), 0xF, 0xF, false);
  }
}
template <int K>
__device__ __forceinline__ float row_readf(float x) {
  return __uint_as_float(row_read<K>(__float_as_uint(x)));
}

// N consecutive words with the widest loads the count allows (the address
// is aligned to the load width by the chunk format).
template <int N>
__device__ __forceinline__ void load_words(const uint8_t* p, uint32_t* out) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int v = 0; v < N / 4; v++) {
      const u32x4_t x = ((g_u32x4_t*)p)[v];
#pragma unroll
      for (int e = 0; e < 4; e++) out[4 * v + e] = x[e];
    }
  } else if constexpr (N % 2 == 0) {
#pragma unroll
    for (int v = 0; v < N / 2; v++) {
      const u32x2_t x = ((g_u32x2_t*)p)[v];
      out[2 * v] = x[0];
      out[2 * v + 1] = x[1];
    }
  } else {
#pragma unroll
    for (int v = 0; v < N; v++) out[v] = ((g_u32_t*)p)[v];
  }
}

// x *= a in place.  The rescale runs in a rarely taken branch; tying the
// product to its source register keeps the compiler from renaming the
// accumulators there and copying them back on the common path.
__device__ __forceinline__ void scale_inplace(f32x4_t& x, float a) {
#pragma unroll
  for (int e = 0; e < 4; e++) asm volatile("v_mul_f32 %0, %1, %0" : "+v"(x[e]) : "v"(a));
}

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
// The low / high element of a word of two values of the cache dtype, and a
// pair packed into one (round to nearest even).
template <int DT>
__device__ __forceinline__ float el_lo(uint32_t w) {
  if constexpr (DT == kF16) return f16_to_f32(static_cast<uint16_t>(w));
  else return bf_lo(w);
}
template <int DT>
__device__ __forceinline__ float el_hi(uint32_t w) {
  if constexpr (DT == kF16) return f16_to_f32(static_cast<uint16_t>(w >> 16));
  else return bf_hi(w);
}
template <int DT>
__device__ __forceinline__ uint32_t pack_el(float a, float b) {
  if constexpr (DT == kF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
  else
    return pack_bf16(a, b);
}
// Two fp32 values rounded to the cache dtype (to nearest even): bf16
// through one v_cvt_pk_bf16_f32 (the software rounding takes about six
// instructions a value).
template <int DT>
__device__ __forceinline__ void round2(float& a, float& b) {
  if constexpr (DT == kBF16) {
    const uint32_t w = pack_bf16(a, b);
    a = bf_lo(w);
    b = bf_hi(w);
  } else {
    a = round_to<DT>(a);
    b = round_to<DT>(b);
  }
}
template <int DT>
__device__ __forceinline__ uint32_t out_el(float x) {
  if constexpr (DT == kF16) return f32_to_f16(x);
  else return f32_to_bf16(x);
}

// One step of the split-K merge (sdpa_vector.h:320-394) over N partials of
// an element: the running (M, L, o) rescaled to the new max, then each live
// partial added with its weight.  qdecode_combine_kernel and the in-launch
// merge both take their partials through this in groups of 4, so the two
// paths round alike (the no-allocation entry point, which has no counters,
// merges in the separate launch and must equal the allocating one).
template <int N, int E>
__device__ __forceinline__ void qmerge_step(float& M, float& L, float (&o)[E], int k0, int K,
                                            const float (&mlm)[N], const float (&mll)[N],
                                            const float (&oo)[N][E]) {
  float mm[N];
  float Mn = M;
#pragma unroll
  for (int q = 0; q < N; q++) {
    mm[q] = k0 + q < K ? mlm[q] : -INFINITY;
    Mn = fmaxf(Mn, mm[q]);
  }
  const float f = M == -INFINITY ? 0.0f : exp2f((M - Mn) * kLog2e);
  L *= f;
#pragma unroll
  for (int e = 0; e < E; e++) o[e] *= f;
#pragma unroll
  for (int q = 0; q < N; q++) {
    // stale slots: weight 0, and their (possibly non-finite) values are
    // selected away rather than multiplied by it
    const bool live = mm[q] != -INFINITY;
    const float w = live ? exp2f((mm[q] - Mn) * kLog2e) : 0.0f;
    L = fmaf(w, live ? mll[q] : 0.0f, L);
#pragma unroll
    for (int e = 0; e < E; e++) o[e] = fmaf(w, live ? oo[q][e] : 0.0f, o[e]);
  }
  M = Mn;
}

// The in-launch merge of NP (sequence, head pair)s' partials (K[p] of pair
// p) by the wave that counted in last for each: the partials come back
// through device-coherent loads (they were stored the same way), every
// pair's first 4 in one round trip, then 4 a round trip; lane l
// takes head l / (64 / HP) and D * HP / 64 consecutive floats of its row,
// whose 8-byte word p holds dims 16 (p / 8) + 4 (p % 4) + 2 ((p / 4) % 2)
// and the next (the order of the decode kernel's coherent stores).
template <int HP, int D, int DT, int NP>
__device__ __forceinline__ void qdecode_merge_pairs(const DecodeArgs& a, const int (&pair)[NP],
                                                    const int (&K)[NP], int lane) {
  constexpr int LPH = 64 / HP, EPL = D / LPH, kQuad = 4;
  static_assert(EPL % 2 == 0, "2-element output stores");
  const int rep = a.rep, n_hg = (rep + HP - 1) / HP, HG = a.Hkv * n_hg;
  const int r = lane / LPH, d0 = (lane % LPH) * EPL;
  // partials k0 .. k0 + 3 of pair p (slots past the count: the last one's,
  // selected away by the merge)
  auto load_quad = [&](int p, int k0, float (&mlm)[kQuad], float (&mll)[kQuad],
                       float (&oo)[kQuad][EPL]) __attribute__((always_inline)) {
    const int64_t slot0 = static_cast<int64_t>(pair[p]) * a.max_parts;
#pragma unroll
    for (int q = 0; q < kQuad; q++) {
      const int64_t slot = (slot0 + min(k0 + q, K[p] - 1)) * HP + r;
      const uint64_t ml = __hip_atomic_load(reinterpret_cast<const uint64_t*>(a.ws_ml) + slot,
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      mlm[q] = __uint_as_float(static_cast<uint32_t>(ml));
      mll[q] = __uint_as_float(static_cast<uint32_t>(ml >> 32));
      const uint64_t* src = reinterpret_cast<const uint64_t*>(a.ws_o + slot * D + d0);
#pragma unroll
      for (int e = 0; e < EPL / 2; e++) {
        const uint64_t x = __hip_atomic_load(src + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        oo[q][2 * e] = __uint_as_float(static_cast<uint32_t>(x));
        oo[q][2 * e + 1] = __uint_as_float(static_cast<uint32_t>(x >> 32));
      }
    }
  };
  float M[NP], L[NP], o[NP][EPL];
  {
    // every pair's first 4 partials in one round trip
    float mlm[NP][kQuad], mll[NP][kQuad], oo[NP][kQuad][EPL];
#pragma unroll
    for (int p = 0; p < NP; p++) load_quad(p, 0, mlm[p], mll[p], oo[p]);
#pragma unroll
    for (int p = 0; p < NP; p++) {
      M[p] = -INFINITY;
      L[p] = 0.0f;
#pragma unroll
      for (int e = 0; e < EPL; e++) o[p][e] = 0.0f;
      qmerge_step<kQuad, EPL>(M[p], L[p], o[p], 0, K[p], mlm[p], mll[p], oo[p]);
    }
  }
#pragma unroll
  for (int p = 0; p < NP; p++) {
    for (int k0 = kQuad; k0 < K[p]; k0 += kQuad) {
      float mlm[kQuad], mll[kQuad], oo[kQuad][EPL];
      load_quad(p, k0, mlm, mll, oo);
      qmerge_step<kQuad, EPL>(M[p], L[p], o[p], k0, K[p], mlm, mll, oo);
    }
    const int seq = pair[p] / HG, j = pair[p] % HG;
    const int64_t hq0 = static_cast<int64_t>(j / n_hg) * rep + (j % n_hg) * HP;
    const int nh = min(HP, rep - (j % n_hg) * HP);
    if (r < nh) {
      const float inv = L[p] > 0.0f ? 1.0f / L[p] : 0.0f;
      uint16_t* dst = a.out + seq * a.o_ss + (hq0 + r) * a.o_sh;
#pragma unroll
      for (int e = 0; e < EPL; e += 2) {
        const int w = (d0 + e) / 2;
        const int d = 16 * (w >> 3) + 4 * (w & 3) + 2 * ((w >> 2) & 1);
        *reinterpret_cast<uint32_t*>(dst + d) =
            out_el<DT>(o[p][e] * inv) | (out_el<DT>(o[p][e + 1] * inv) << 16);
      }
    }
  }
}

// The decode token t of (sequence seq, kv head hk) -- the key and value
// rows the router hands over with the attention, [seq][kv head][D] -- into
// its pool block, quantized as the paged append quantizes it
// (affine_quantize8, group 64; updateQuantized, KVCache.swift:1049-1122):
// lanes 0 .. D/8 - 1 take 8 dims of the key row each, the next D/8 lanes
// the value row's, 8 lanes a group.  Stores as the append's: key code
// words, value code bytes (8-bit) or nibbles merged into their words with
// atomics (4-bit: a word holds 8 tokens of a dim), scale and bias by a
// group's first lane.
template <int BITS, int D, int DT>
__device__ __forceinline__ void qdecode_write_token(const DecodeArgs& a, int seq, int hk, int t,
                                                    int lane) {
  using E = Elem<DT>;
  constexpr int LPR = D / 8, G = D / 64;
  const bool active = lane < 2 * LPR;
  const int which = lane / LPR, j8 = lane % LPR;
  // the token's block, read beside its rows (not after the quantization)
  const int64_t blk = a.table[static_cast<int64_t>(seq) * a.table_stride + t / a.block_size];
  float v[8];
  if (active) {
    const uint16_t* src = which ? a.new_v + seq * a.nv_ss + hk * a.nv_sh
                                : a.new_k + seq * a.nk_ss + hk * a.nk_sh;
    const u32x4_t x = *(g_u32x4_t*)(src + 8 * j8);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[2 * e] = el_lo<DT>(x[e]);
      v[2 * e + 1] = el_hi<DT>(x[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = 0.0f;
  }
  uint32_t code[8];
  float scale, bias;
  affine_quantize8<DT, BITS, 64>(v, code, scale, bias);  // (every lane: team shuffles)
  if (!active) return;
  const int tib = t % a.block_size;
  // (the pool is written through the view's base, which the decode only reads elsewhere)
  uint8_t* chunk = const_cast<uint8_t*>(a.base) + blk * a.block_bytes + hk * a.head_bytes;
  uint8_t* c = chunk + (which ? a.vc_off : a.kc_off);
  if (!which) {
    if constexpr (BITS == 4) {
      uint32_t w = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) w |= code[i] << (4 * i);
      *reinterpret_cast<uint32_t*>(c + qk_word_off(tib, j8, D, 4)) = w;
    } else {
      *reinterpret_cast<uint32_t*>(c + qk_word_off(tib, 2 * j8, D, 8)) =
          code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
      *reinterpret_cast<uint32_t*>(c + qk_word_off(tib, 2 * j8 + 1, D, 8)) =
          code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      int sh;
      const int64_t off = qv_word_off(tib, 8 * j8 + i, D, BITS, &sh);
      if constexpr (BITS == 8) {
        c[off + sh / 8] = static_cast<uint8_t>(code[i]);
      } else {
        uint32_t* word = reinterpret_cast<uint32_t*>(c + off);
        atomicAnd(word, ~(0xFu << sh));
        atomicOr(word, code[i] << sh);
      }
    }
  }
  if (j8 % 8 == 0) {
    typename E::T* sbp = reinterpret_cast<typename E::T*>(chunk + a.sb_off);
    sbp[qsb_index(tib, which, j8 / 8, 0, G, false)] = E::from_f32(scale);
    sbp[qsb_index(tib, which, j8 / 8, 1, G, false)] = E::from_f32(bias);
  }
}

// Orders one wave's LDS writes before its later LDS reads by other lanes
// (no workgroup barrier: every workgroup is a single wave).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Inclusive prefix sum over the 64 lanes of a wave: DPP row shifts within
// each row of 16 lanes, then the totals of the rows before.
__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31);
  const int r2 = __builtin_amdgcn_readlane(x, 47);
  return x + (lane >= 16 ? r0 : 0) + (lane >= 32 ? r1 : 0) + (lane >= 48 ? r2 : 0);
}

// Maximum over the 64 lanes of a wave (a scalar).
__device__ __forceinline__ int wave_max(int x) {
  x = max(x, static_cast<int>(row_read<8>(static_cast<uint32_t>(x))));
  x = max(x, static_cast<int>(row_read<4>(static_cast<uint32_t>(x))));
  x = max(x, static_cast<int>(row_read<2>(static_cast<uint32_t>(x))));
  x = max(x, static_cast<int>(row_read<1>(static_cast<uint32_t>(x))));
  return max(max(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
             max(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

// Lane s % 64 of register s / 64 of a per-sequence table held in NR
// registers (s uniform).
template <int NR>
__device__ __forceinline__ int seq_at(const int (&t)[NR], int s) {
  int v = __builtin_amdgcn_readlane(t[0], s & 63);
#pragma unroll
  for (int r = 1; r < NR; r++)
    if ((s >> 6) == r) v = __builtin_amdgcn_readlane(t[r], s & 63);
  return v;
}

// GR: the quantization group in 64-dim units (1: group 64; 2: group 128,
// whose scale and bias serve two consecutive 64-dim groups of the kernel)
template <int BITS, int D, int HP, int DT = kBF16, int GR = 1>
struct QD {
  static constexpr int G = D / 64;            // 64-dim groups per row
  static constexpr int PP = 16 / HP;          // token parts of a score tile
  static constexpr int TT = 4 / PP;           // score tiles per 64-token step
  static constexpr int SPW = 4 / PP;          // lane groups per part
  static constexpr int SL = D * PP / 32;      // score K slices (8 dims per lane)
  static constexpr int UW = BITS / 4;         // words per 8-dim unit
  static constexpr int RUN = (D / 32) * UW;   // key words of one lane-group run
  static constexpr int NT = D / 16;           // 16-dim output tiles
  static constexpr int VW = NT * UW;          // value words per lane per sub-block
  static constexpr int ROW = D * BITS / 8;    // key code bytes per token
  static constexpr int SBW = 2 * G / GR;      // scale/bias words per token (K, V)
  static_assert(G % GR == 0, "whole quantization groups per row");
  static constexpr int QROW = 16 * SPW + 1;   // query-table entries per slice
  static constexpr int QCH = HP * D / 8;      // 8-dim query chunks of a head group
  static constexpr int QPL = (QCH + 63) / 64; // query chunks per lane
  static constexpr float MAG = (BITS == 4) ? 128.0f : 2176.0f;   // value operands
  static constexpr float KMAG = (BITS == 4) ? 16.0f : (DT == kF16 ? 256.0f : 272.0f);  // key operands
  static constexpr float C0 = (BITS == 4) ? 8.0f : 128.0f;
  // per-step operand registers; steps are double buffered when they fit
  static constexpr int BUF = D * UW / 4 + HP * D / 32;
  static constexpr bool kPrefetch = BUF <= 48;
  // one wave per SIMD (D = 256) with 4 heads per part: the next step's key
  // words and scales load while a step computes, its value words at the
  // step's start (behind the scores); whole double buffers would not fit
  // beside the rest, and with 8 heads per part neither does this (it
  // spills).  (At D 128, 8-bit, where two waves share a SIMD, it fits but
  // measured no faster: the partner wave already covers the loads.)  f16
  // caches at 8 bits hold more live registers here (their f16 query and
  // key operands): with the prefetch they spill to scratch inside the loop,
  // so they load then compute.
  static constexpr bool kPrefetchK =
      !kPrefetch && D >= 256 && HP == 4 && !(DT == kF16 && BITS == 8);

  struct Buf {
    uint32_t kw[TT][PP][RUN];    // key words of this lane's token, per tile
    uint32_t sb[TT][4][SBW];     // scale/bias of the 4 scored tokens, per tile
    uint32_t vw[2][VW];          // value words, per 32-token sub-block
    uint32_t wt[TT][2];          // stored bf16 weights of the 4 tokens (weights mode)
  };
};

// Waves per workgroup.  Up to D = 128 two waves share each SIMD (256 VGPRs
// each) and a workgroup is the 8 waves of one CU, so that the two waves of a
// SIMD can balance their progress; D = 256 runs one wave per SIMD.
template <int D>
constexpr int qd_waves() { return D >= 256 ? 1 : 8; }

// Kernel modes: the fused single pass (scores, online fp32 softmax, P.V),
// or the two matrix-core passes of the reference-arithmetic path: the
// bf16 scores written to score rows (kModeScores), and, after the
// reference softmax has turned them into bf16 weights in place, P.V from
// the stored weights (kModeWeights: no key loads, no score MFMAs, no max;
// the partials are plain sums, merged with max 0 and the pair's first
// partial carrying sum 1).  kModeFusedG128 is the fused pass over caches
// quantized with group 128 (GenerateParameters.kvGroupSize,
// Evaluate.swift:109-112): each scale / bias pair is read once for two
// 64-dim groups; the decode token is left to the append launch.
constexpr int kModeFused = 0, kModeScores = 1, kModeWeights = 2, kModeFusedG128 = 3;

// See the header comment for the work split.  Every wave works on its own
// range with its own LDS tables; the waves of a workgroup only share their
// SIMD placement and unit counters.
template <int BITS, int D, int HP, int MODE, int DT>
__global__ void __launch_bounds__(64 * qd_waves<D>())
__attribute__((amdgpu_waves_per_eu((D >= 256) ? 1 : 2)))
qdecode_kernel(DecodeArgs a) {
  constexpr bool kFused = MODE == kModeFused || MODE == kModeFusedG128;
  constexpr int GR = MODE == kModeFusedG128 ? 2 : 1;
  static_assert(DT == kBF16 || kFused, "the reference modes store bf16 rows");
  using C = QD<BITS, D, HP, DT, GR>;
  constexpr int WPG = qd_waves<D>();
  constexpr int G = C::G, PP = C::PP, TT = C::TT, SPW = C::SPW, SL = C::SL;
  constexpr int RUN = C::RUN, NT = C::NT, VW = C::VW, ROW = C::ROW, SBW = C::SBW;
  constexpr int QROW = C::QROW, QCH = C::QCH, QPL = C::QPL;
  constexpr float MAG = C::MAG, KMAG = C::KMAG, C0 = C::C0;
  using Buf = typename C::Buf;
  constexpr int QT_ENTRIES = SL * QROW;
  static_assert(QT_ENTRIES * 16 >= kMaxSeqs * 8, "the sequence scan reuses the query table");

  // LDS (one set per wave): the score B operands, the KV chunk of every
  // 32-token sub-block of the range, and the range's segments.  The
  // per-sequence unit prefix of the set-up lives in the query table's space.
  __shared__ u32x4_t qtab_g[WPG][QT_ENTRIES];
  __shared__ int64_t sub_off_g[WPG][2 * kMaxRange];  // chunk byte offset (block, kv head)
  __shared__ int32_t sub_t0_g[WPG][2 * kMaxRange];   // first token of the sub-block in its block
  // per segment: seq, pair, first step, steps, len, first unit of the range,
  // cost position of the pair's first step
  __shared__ int32_t seg_tab_g[WPG][kMaxRange][7];
  __shared__ int32_t simd_of[WPG];  // SIMD of each wave of the workgroup
  __shared__ int32_t done_of[WPG];  // units each wave has started
  // score / weight rows (score and weights modes): per unit, the element
  // offset of its head group's first row at the unit's first token, and the
  // group's live heads
  __shared__ int64_t u_woff_g[!kFused ? WPG : 1][!kFused ? kMaxRange : 1];
  __shared__ int32_t u_nh_g[!kFused ? WPG : 1][!kFused ? kMaxRange : 1];
  const int wv = WPG > 1 ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6) : 0;
  u32x4_t* qtab = qtab_g[wv];
  int64_t* sub_off = sub_off_g[wv];
  int32_t* sub_t0 = sub_t0_g[wv];
  int32_t(*seg_tab)[7] = seg_tab_g[wv];

  const int lane = threadIdx.x & 63, n = lane & 15, lg = lane >> 4;
  const int w = blockIdx.x * WPG + wv, W = gridDim.x * WPG;
  const int ns = a.n_seqs;

  // ---- sequence lengths first (the set-up is a chain of dependent loads):
  // lane l of register r holds sequence 64 r + l
  constexpr int SR = kMaxSeqs / 64;
  int len_r[SR];
#pragma unroll
  for (int r = 0; r < SR; r++) {
    const int s = 64 * r + lane;
    len_r[r] = 0;
    if (64 * r < ns) len_r[r] = (s < ns) ? (a.seq_lens ? a.seq_lens[s] : a.max_len) : 0;
  }

  // The wave that shares this wave's SIMD (-1: none).  Of two waves on a
  // SIMD the older one wins instruction issue, so left alone it finishes
  // its range long before the younger one, which then runs alone; instead
  // the wave that is behind raises its priority (below).
  int partner = -1;
  if constexpr (WPG > 1) {
    uint32_t hw_id;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw_id));
    simd_of[wv] = (hw_id >> 4) & 3;  // HW_ID[5:4]: SIMD
    done_of[wv] = 0;
    // LDS-only fences: the length loads stay in flight across the barrier
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    for (int o = 0; o < WPG; o++)
      if (o != wv && simd_of[o] == simd_of[wv]) partner = o;
    partner = __builtin_amdgcn_readfirstlane(partner);
  }
  const int rep = a.rep, n_hg = (rep + HP - 1) / HP, HG = a.Hkv * n_hg;
  const int subs = a.block_size >> 5;  // 32-token sub-blocks per pool block
  // this lane's roles: score column (part p, head h); key-operand lane
  // group (part pA, unit slot wA)
  const int p = n / HP, h = n % HP;
  const int pA = lg / SPW, wA = lg % SPW;

  // ---- cost per sequence ((steps + kSegCost) x head pairs) and its prefix
  // sums, in registers like the lengths; a pair's cost units are kSegCost
  // lead-in units, then its steps
  int cum_r[SR], nst_r[SR];
  int carry = 0, max_nst = 0;
#pragma unroll
  for (int r = 0; r < SR; r++) {
    cum_r[r] = 0;
    nst_r[r] = 0;
    if (64 * r < ns) {
      const int nst = (len_r[r] + 63) >> 6;
      const int cost = nst > 0 ? (nst + kSegCost) * HG : 0;
      const int incl = wave_incl_scan(cost, lane);
      cum_r[r] = carry + incl - cost;
      nst_r[r] = nst;
      carry += __builtin_amdgcn_readlane(incl, 63);
      max_nst = max(max_nst, nst);
    }
  }
  max_nst = wave_max(max_nst);
  const int U = __builtin_amdgcn_readfirstlane(carry);
  if (MODE != kModeScores && w == 0) {  // empty sequences: zero output
#pragma unroll
    for (int r = 0; r < SR; r++) {
      uint64_t empty = __builtin_amdgcn_ballot_w64(64 * r + lane < ns && nst_r[r] == 0);
      while (empty) {
        const int s = 64 * r + __builtin_ctzll(empty);
        empty &= empty - 1;
        for (int idx = lane; idx < a.Hq * D; idx += 64)
          a.out[s * a.o_ss + (idx / D) * a.o_sh + idx % D] = 0;
      }
    }
  }
  // cost units per wave: W ranges (<= kMaxRange units, by the host's
  // choice of W), and at least max_nst / (max_parts - 1) so that no pair is
  // split into more than max_parts partials (the host's choice of max_parts
  // keeps that within kMaxRange)
  const int cper = max((U + W - 1) / W, (max_nst + a.max_parts - 2) / (a.max_parts - 1));
  // sequence lengths past the view's max_len (a broken call) would need
  // longer ranges than the LDS tables hold: write nothing rather than past them
  if (cper > kMaxRange) return;
  const int u0 = w * cper;
  if (u0 >= U) return;
  const int u1 = min(U, u0 + cper);

  // ---- the range's segments: maximal runs of steps in one (seq, pair); the
  // range's steps are its units 0 .. nunits - 1.  The walk runs on scalars;
  // lane e of the block-table slice (below) picks the segment of its unit
  // e / 2 on the way (units past the range map to the range's last unit).
  int nseg = 0, nunits = 0;
  int sel_seq[2] = {0, 0}, sel_j[2] = {0, 0}, sel_step[2] = {0, 0}, sel_len[2] = {1, 1};
  int seq0 = 0, j0 = 0;  // the first segment's (sequence, pair)
  {
    // the last sequence whose prefix is <= u0
    int cnt = 0;
#pragma unroll
    for (int r = 0; r < SR; r++)
      cnt += __popcll(__builtin_amdgcn_ballot_w64(64 * r + lane < ns && cum_r[r] <= u0));
    int ss = max(cnt - 1, 0), u = u0;
    while (u < u1) {
      while (ss < ns - 1 && seq_at(nst_r, ss) == 0) ss++;
      const int nst = max(seq_at(nst_r, ss), 1), per = nst + kSegCost;
      const int cum = seq_at(cum_r, ss), len = seq_at(len_r, ss);
      const int local = u - cum;
      const int j = local / per, t = local % per - kSegCost;  // t < 0: lead-in
      const int t0 = max(t, 0);
      const int take = min(nst, t + (u1 - u)) - t0;
      if (take > 0) {
        if (lane == 0) {
          seg_tab[nseg][0] = ss;
          seg_tab[nseg][1] = j;
          seg_tab[nseg][2] = t0;
          seg_tab[nseg][3] = take;
          seg_tab[nseg][4] = len;
          seg_tab[nseg][5] = nunits;
          seg_tab[nseg][6] = cum + j * per + kSegCost;
        }
        if (nseg == 0) {
          seq0 = ss;
          j0 = j;
        }
#pragma unroll
        for (int r = 0; r < 2; r++) {
          const int ui = (lane + 64 * r) >> 1;
          const bool sel = ui >= nunits;
          sel_seq[r] = sel ? ss : sel_seq[r];
          sel_j[r] = sel ? j : sel_j[r];
          sel_step[r] = sel ? t0 + min(ui - nunits, take - 1) : sel_step[r];
          sel_len[r] = sel ? len : sel_len[r];
        }
        nseg++;
        nunits += take;
      }
      u += per - (t + kSegCost);  // on to the next pair
      if (j == HG - 1) ss++;
    }
  }
  if (nunits == 0) return;  // the range holds lead-in units only

  // ---- block-table slice: the chunk of each sub-block of the range.  These
  // loads, then the first segment's queries, are issued before any KV load
  // (global loads complete in issue order, so later set-up loads would wait
  // for the KV data).
  int64_t my_off[2];
  int32_t my_t0[2];
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const int e = lane + 64 * r;
    const int nsub = (sel_len[r] + 31) >> 5;
    const int sbi = max(min(2 * sel_step[r] + (e & 1), nsub - 1), 0);
    const int64_t blk = a.table[static_cast<int64_t>(sel_seq[r]) * a.table_stride + sbi / subs];
    my_off[r] = blk * a.block_bytes + static_cast<int64_t>(sel_j[r] / n_hg) * a.head_bytes;
    my_t0[r] = (sbi % subs) * 32;
  }
  // (The lambdas below are forced inline: called from several places, the
  // compiler would otherwise outline them as functions.)
  // queries of the head group of pair j of sequence seq: 8 dims (16 bytes)
  // per chunk
  auto load_q_sj = [&](int seq, int j, u32x4_t* qr) __attribute__((always_inline)) {
    const int64_t hq0 = static_cast<int64_t>(j / n_hg) * rep + (j % n_hg) * HP;
    const int nh = min(HP, rep - (j % n_hg) * HP);
#pragma unroll
    for (int c = 0; c < QPL; c++) {
      const int ci = min(lane + 64 * c, QCH - 1), r = min(ci / (D / 8), nh - 1);
      qr[c] = *(g_u32x4_t*)(a.q + seq * a.q_ss + (hq0 + r) * a.q_sh + 8 * (ci % (D / 8)));
    }
  };
  // ... of segment k
  auto load_q = [&](int k, u32x4_t* qr) __attribute__((always_inline)) {
    load_q_sj(__builtin_amdgcn_readfirstlane(seg_tab[k][0]), __builtin_amdgcn_readfirstlane(seg_tab[k][1]), qr);
  };
  u32x4_t qpre[QPL];
  if constexpr (MODE != kModeWeights) load_q_sj(seq0, j0, qpre);
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const int e = lane + 64 * r;
    if (e < 2 * kMaxRange) {
      sub_off[e] = my_off[r];
      sub_t0[e] = my_t0[r];
    }
    if constexpr (!kFused) {
      if ((e & 1) == 0 && e < 2 * kMaxRange) {
        const int j = sel_j[r];
        const int64_t hq0 = static_cast<int64_t>(j / n_hg) * rep + (j % n_hg) * HP;
        u_woff_g[wv][e >> 1] = (static_cast<int64_t>(sel_seq[r]) * a.Hq + hq0) * a.sc_stride +
                               static_cast<int64_t>(sel_step[r]) * 64;
        u_nh_g[wv][e >> 1] = min(HP, rep - (j % n_hg) * HP);
      }
    }
  }
  // the zero entry of every query-table slice (lanes outside a column's part)
  for (int sg = lane; sg < SL; sg += 64) qtab[sg * QROW + 16 * SPW] = u32x4_t{0u, 0u, 0u, 0u};
  wave_lds_sync();

  // ---- the router's decode step (updateQuantized, then the attention):
  // the token of every pair whose last step this range holds goes into its
  // block before any of the range's loads, and is complete (at the L2 this
  // wave reads from) before they issue, so the unit holding it reads it back.
  // The unit is this wave's alone, as are the blocks it reads (the host
  // passes the token only with one head group per kv head, so no other
  // wave writes the same words).
  if constexpr (MODE == kModeFused) {
    if (a.new_k) {
      bool wrote = false;
      for (int kk = 0; kk < nseg; kk++) {
        const int len = __builtin_amdgcn_readfirstlane(seg_tab[kk][4]);
        const int t0 = __builtin_amdgcn_readfirstlane(seg_tab[kk][2]);
        const int take = __builtin_amdgcn_readfirstlane(seg_tab[kk][3]);
        if (len <= 0 || t0 + take != (len + 63) >> 6) continue;
        qdecode_write_token<BITS, D, DT>(a, __builtin_amdgcn_readfirstlane(seg_tab[kk][0]),
                                         __builtin_amdgcn_readfirstlane(seg_tab[kk][1]) / n_hg,
                                         len - 1, lane);
        wrote = true;
      }
      if (wrote) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
  }

  // ---- per-unit loads
  // This lane's byte offsets from a 32-token sub-block's two scalar bases
  // (codes: chunk + first token * ROW; scale/bias: chunk + first token *
  // SBW * 4); tile tau's key row and scored tokens sit in sub-block ks / ss.
  int32_t k_lane[TT], sb_lane[TT];
  int ks_sub[TT], ss_sub[TT];
#pragma unroll
  for (int tau = 0; tau < TT; tau++) {
    const int c = tau * PP + pA, c2 = tau * PP + p;
    ks_sub[tau] = c >> 1;
    k_lane[tau] = a.kc_off + (8 * (n >> 2) + tok_off<BITS>(c & 1, n & 3)) * ROW + wA * RUN * 4;
    ss_sub[tau] = c2 >> 1;
    sb_lane[tau] = a.sb_off + (8 * lg + tok_off<BITS>(c2 & 1, 0)) * SBW * 4;
  }
  const int32_t v_lane = a.vc_off + (lg * 16 + n) * VW * 4;
  // code and scale/bias bases of unit ui's two 32-token sub-blocks
  auto step_bases = [&](int ui, const uint8_t** bc, const uint8_t** bs) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const uint8_t* cb = a.base + __builtin_amdgcn_readfirstlane(sub_off[2 * ui + s]);
      const int t0 = __builtin_amdgcn_readfirstlane(sub_t0[2 * ui + s]);
      bc[s] = cb + t0 * ROW;
      bs[s] = cb + t0 * SBW * 4;
    }
  };
  // the first of a lane's 4 tokens within a step, per tile (its pairs are
  // t, t + 1 and t + 4, t + 5 at 4 bits; t .. t + 3 at 8 bits)
  int32_t w_tok[TT];
#pragma unroll
  for (int tau = 0; tau < TT; tau++) {
    const int c = tau * PP + p;
    w_tok[tau] = 32 * (c >> 1) + 8 * lg + tok_off<BITS>(c & 1, 0);
  }
  // this lane's score / weight row offset within its unit's head group (a
  // head past the group's live heads reads the last live one)
  auto w_row = [&](int nh_u) __attribute__((always_inline)) {
    return static_cast<int64_t>(min(h, nh_u - 1)) * a.sc_stride;
  };
  // key words (stored weights in the weights mode) and scales / biases of unit ui
  auto load_k = [&](int ui, Buf& b) __attribute__((always_inline)) {
    const uint8_t* bc[2];
    const uint8_t* bs[2];
    step_bases(ui, bc, bs);
    if constexpr (MODE == kModeWeights) {
      const int64_t wo = u_woff_g[wv][ui] + w_row(u_nh_g[wv][ui]);
#pragma unroll
      for (int tau = 0; tau < TT; tau++) {
        const uint16_t* wp = a.sc + wo + w_tok[tau];
        if constexpr (BITS == 4) {
          b.wt[tau][0] = *(g_u32_t*)wp;
          b.wt[tau][1] = *(g_u32_t*)(wp + 4);
        } else {
          const u32x2_t x = *(g_u32x2_t*)wp;
          b.wt[tau][0] = x[0];
          b.wt[tau][1] = x[1];
        }
      }
    }
#pragma unroll
    for (int tau = 0; tau < TT; tau++) {
      if constexpr (MODE != kModeWeights) {
        const uint8_t* row = (ks_sub[tau] ? bc[1] : bc[0]) + k_lane[tau];
#pragma unroll
        for (int rho = 0; rho < PP; rho++) load_words<RUN>(row + rho * SPW * RUN * 4, b.kw[tau][rho]);
      }
      const uint8_t* sbp = (ss_sub[tau] ? bs[1] : bs[0]) + sb_lane[tau];
#pragma unroll
      for (int i = 0; i < 4; i++)
        load_words<SBW>(sbp + (tok_off<BITS>(0, i) - tok_off<BITS>(0, 0)) * SBW * 4, b.sb[tau][i]);
    }
  };
  // value words of unit ui (none in the score mode)
  auto load_v = [&](int ui, uint32_t (&vw)[2][VW]) __attribute__((always_inline)) {
    if constexpr (MODE != kModeScores) {
      const uint8_t* bc[2];
      const uint8_t* bs[2];
      step_bases(ui, bc, bs);
#pragma unroll
      for (int s = 0; s < 2; s++) load_words<VW>(bc[s] + v_lane, vw[s]);
    }
  };
  auto load_step = [&](int ui, Buf& b) __attribute__((always_inline)) {
    load_k(ui, b);
    load_v(ui, b.vw);
  };

  Buf bufA, bufB;
  uint32_t vcur[2][VW];  // kPrefetchK: the current unit's value words
  if constexpr (C::kPrefetchK)
    load_k(0, bufA);
  else
    load_step(0, bufA);
  const Magic mg;
  const float scale_t = round_to<DT>(a.scale);

  // ---- segment state
  int k = 0;             // current segment
  int seg_seq = 0, seg_j = 0, seg_t = 0, seg_take = 0, seg_len = 0, seg_first = 0, seg_pa = 0, nh = 0;
  // in-launch merge: the (pair, partial count) of the partials this wave
  // counts in at its end, at most two (only a range's first and last
  // segments can be parts of a pair)
  int pend_pair0 = -1, pend_k0 = 0, pend_pair1 = -1, pend_k1 = 0;
  const bool merge_here = kFused && D <= 128 && a.counters != nullptr;
  float sq[G];
  // query table of segment kk from its prefetched chunks: entry (slice sg,
  // column nn, unit slot ws) holds unit sg * SPW + ws of head nn % HP in the
  // key operand's K order; sq = each head's bf16 query sum per group
  auto setup_segment = [&](int kk, const u32x4_t* qr) __attribute__((always_inline)) {
    seg_seq = __builtin_amdgcn_readfirstlane(seg_tab[kk][0]);
    seg_j = __builtin_amdgcn_readfirstlane(seg_tab[kk][1]);
    seg_t = __builtin_amdgcn_readfirstlane(seg_tab[kk][2]);
    seg_take = __builtin_amdgcn_readfirstlane(seg_tab[kk][3]);
    seg_len = __builtin_amdgcn_readfirstlane(seg_tab[kk][4]);
    seg_first = __builtin_amdgcn_readfirstlane(seg_tab[kk][5]);
    seg_pa = __builtin_amdgcn_readfirstlane(seg_tab[kk][6]);
    nh = min(HP, rep - (seg_j % n_hg) * HP);
    if constexpr (MODE == kModeWeights) return;  // no queries: the weights are stored
    float part[QPL][G];
#pragma unroll
    for (int c = 0; c < QPL; c++) {
      const int ci = lane + 64 * c;
      const int r = ci / (D / 8), unit = ci % (D / 8);
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        v[2 * e] = el_lo<DT>(qr[c][e]) * scale_t;
        v[2 * e + 1] = el_hi<DT>(qr[c][e]) * scale_t;
        round2<DT>(v[2 * e], v[2 * e + 1]);
      }
      const bool live = ci < QCH && r < nh;
      float sum = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        v[e] = live ? v[e] : 0.0f;
        sum += v[e];
      }
      u32x4_t ent;
#pragma unroll
      for (int pr = 0; pr < 4; pr++)
        ent[pr] = pack_el<DT>(v[kslot<BITS>(2 * pr)], v[kslot<BITS>(2 * pr + 1)]);
      if (ci < QCH) {
        const int sg = unit / SPW, ws = unit % SPW;
#pragma unroll
        for (int pp = 0; pp < PP; pp++) qtab[sg * QROW + (r + pp * HP) * SPW + ws] = ent;
      }
      // group sums: the 8 chunks of a (head, group) are 8 adjacent lanes
      sum += __shfl_xor(sum, 1);
      sum += __shfl_xor(sum, 2);
      sum += __shfl_xor(sum, 4);
#pragma unroll
      for (int g = 0; g < G; g++) {
        const int src = h * (D / 8) + 8 * g;  // chunk holding (head h, group g)
        const float x = __shfl(sum, src % 64);
        part[c][g] = (src / 64 == c) ? x : 0.0f;
      }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
      sq[g] = 0.0f;
#pragma unroll
      for (int c = 0; c < QPL; c++) sq[g] += part[c][g];
    }
    wave_lds_sync();
  };
  setup_segment(0, qpre);
  // the next segment's queries load while this segment's units compute
  if constexpr (MODE != kModeWeights) load_q(min(1, nseg - 1), qpre);

  f32x4_t oacc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) oacc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f, corr[G];
#pragma unroll
  for (int g = 0; g < G; g++) corr[g] = 0.0f;
  const u32x4_t* qlane = qtab + ((pA == p) ? n * SPW + wA : 16 * SPW);

  auto compute_step = [&](int stp, const Buf& b, const uint32_t (&vw)[2][VW]) __attribute__((always_inline)) {
    const int len = seg_len;
    // ---- scores: acc[tau][g] = q . (KMAG + c) over group g's dims
    f32x4_t acc[TT][G];
#pragma unroll
    for (int tau = 0; tau < TT; tau++)
#pragma unroll
      for (int g = 0; g < G; g++) acc[tau][g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // query slices are read kQA ahead of their MFMAs; the scheduling
    // barrier keeps the compiler from issuing every slice's LDS read up front
    constexpr int kQA = SL < 4 ? SL : 4;
    u32x4_t qring[kQA];
    // slices in group-interleaved order, so consecutive MFMAs feed
    // independent accumulators
    auto slice = [](int o) { return (o % G) * (SL / G) + o / G; };
#pragma unroll
    for (int jj = 0; jj < kQA; jj++) qring[jj] = qlane[slice(jj) * QROW];
#pragma unroll
    for (int o = 0; o < (MODE == kModeWeights ? 0 : SL); o++) {
      const int sg = slice(o);
      const u32x4_t qb = qring[o % kQA];
      if (o + kQA < SL) qring[o % kQA] = qlane[slice(o + kQA) * QROW];
      const int g = sg / (SL / G), rho = sg % PP, kq = sg / PP;
#pragma unroll
      for (int tau = 0; tau < TT; tau++) {
        if constexpr (DT == kF16 && BITS == 4) {
          acc[tau][g] = mfma_qk<DT>(nib_magic_k16(b.kw[tau][rho][kq]), qb, acc[tau][g]);
        } else if constexpr (DT == kF16) {
          acc[tau][g] = mfma_qk<DT>(byte_magic_k16(b.kw[tau][rho][2 * kq], b.kw[tau][rho][2 * kq + 1]),
                                    qb, acc[tau][g]);
        } else if constexpr (BITS == 4) {
          acc[tau][g] = mfma(nib_magic_k(b.kw[tau][rho][kq], mg), qb, acc[tau][g]);
        } else {
          u32x4_t lo, hi;
          byte_magic_k(b.kw[tau][rho][2 * kq], b.kw[tau][rho][2 * kq + 1], mg, lo, hi);
          acc[tau][g] = mfma(lo, qb, acc[tau][g]);
          acc[tau][g] = mfma(hi, qb, acc[tau][g]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    float sc[TT][4], vs[TT][4][G], vb[TT][4][G];
#pragma unroll
    for (int tau = 0; tau < TT; tau++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float s = 0.0f;
#pragma unroll
        for (int g = 0; g < G; g++) {
          const uint32_t kwd = b.sb[tau][i][g / GR], vwd = b.sb[tau][i][(G + g) / GR];
          if constexpr (MODE != kModeWeights) {
            const float ks = el_lo<DT>(kwd);
            s = fmaf(fmaf(-KMAG, ks, el_hi<DT>(kwd)), sq[g], s);
            s = fmaf(ks, acc[tau][g][i], s);
          }
          vs[tau][i][g] = el_lo<DT>(vwd);
          vb[tau][i][g] = el_hi<DT>(vwd);
        }
        if constexpr (MODE == kModeWeights) {
          // the stored weight of token i: pairs (i0, i2) and (i1, i3) share a word
          const uint32_t wd = b.wt[tau][i & 1];
          sc[tau][i] = (i >> 1) ? bf_hi(wd) : bf_lo(wd);
        } else {
          sc[tau][i] = s;
        }
      }
    if constexpr (MODE != kModeWeights) {
      // the reference stores the scores in the query dtype before the
      // softmax (quantizedMM returns T, KVCache.swift:1945-1949)
#pragma unroll
      for (int tau = 0; tau < TT; tau++) {
        round2<DT>(sc[tau][0], sc[tau][1]);
        round2<DT>(sc[tau][2], sc[tau][3]);
      }
    }
    if (stp * 64 + 64 > len) {  // the sequence ends inside this step
      // a real branch: the masked values leave through the asm statements,
      // so the selects cannot be hoisted onto the common path
#pragma unroll
      for (int tau = 0; tau < TT; tau++) {
        const int c = tau * PP + p, s = c >> 1, q = c & 1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const bool ok = stp * 64 + 32 * s + 8 * lg + tok_off<BITS>(q, i) < len;
          sc[tau][i] = ok ? sc[tau][i] : (MODE == kModeWeights ? 0.0f : -INFINITY);
          asm volatile("" : "+v"(sc[tau][i]));
#pragma unroll
          for (int g = 0; g < G; g++) {
            vs[tau][i][g] = ok ? vs[tau][i][g] : 0.0f;
            vb[tau][i][g] = ok ? vb[tau][i][g] : 0.0f;
            asm volatile("" : "+v"(vs[tau][i][g]), "+v"(vb[tau][i][g]));
          }
        }
      }
    }

    if constexpr (MODE == kModeScores) {
      // the bf16 scores of head h's row at this lane's 4 tokens (past the
      // sequence -inf, inside the row's padding)
      if (h < nh) {
        uint16_t* row = a.sc + (static_cast<int64_t>(seg_seq) * a.Hq +
                                static_cast<int64_t>(seg_j / n_hg) * rep + (seg_j % n_hg) * HP + h) *
                                   a.sc_stride + stp * 64;
#pragma unroll
        for (int tau = 0; tau < TT; tau++) {
          const uint32_t w0 = pack_bf16(sc[tau][0], sc[tau][2]);
          const uint32_t w1 = pack_bf16(sc[tau][1], sc[tau][3]);
          if constexpr (BITS == 4) {
            *reinterpret_cast<uint32_t*>(row + w_tok[tau]) = w0;
            *reinterpret_cast<uint32_t*>(row + w_tok[tau] + 4) = w1;
          } else {
            *reinterpret_cast<u32x2_t*>(row + w_tok[tau]) = u32x2_t{w0, w1};
          }
        }
      }
      return;
    }
    float pr[TT][4];
    if constexpr (MODE == kModeWeights) {
#pragma unroll
      for (int tau = 0; tau < TT; tau++)
#pragma unroll
        for (int i = 0; i < 4; i++) pr[tau][i] = sc[tau][i];
    } else {
    // ---- online softmax with a lazily refreshed max
    float mx = -INFINITY;
#pragma unroll
    for (int tau = 0; tau < TT; tau++)
#pragma unroll
      for (int i = 0; i < 4; i++) mx = fmaxf(mx, sc[tau][i]);
    if (__builtin_amdgcn_ballot_w64(mx > m_run + kTau)) {
      // max over the lanes of head h: the other parts of the row, other rows
#pragma unroll
      for (int o = HP; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const bool up = mx > m_run + kTau;
      const float alpha = up ? (m_run == -INFINITY ? 0.0f : exp2f((m_run - mx) * kLog2e)) : 1.0f;
      m_run = up ? mx : m_run;
      l_run *= alpha;
#pragma unroll
      for (int g = 0; g < G; g++) corr[g] *= alpha;
      // the P.V accumulators of lane n + 16 lg carry head n = h for n < HP;
      // a new segment starts with m_run = -inf, so alpha = 0 also clears them
#pragma unroll
      for (int t = 0; t < NT; t++) scale_inplace(oacc[t], alpha);
    }
    const float m2 = fmaxf(m_run * kLog2e, -3.402823466e38f);
#pragma unroll
    for (int tau = 0; tau < TT; tau++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        pr[tau][i] = fast_exp2(fmaf(sc[tau][i], kLog2e, -m2));
        l_run += pr[tau][i];
      }
    }

    // ---- P = p * s_v as bf16 hi + lo pairs, in value-operand register order
    uint32_t pk[TT][2][G][2];  // [tile][pair][group][hi, lo]
#pragma unroll
    for (int tau = 0; tau < TT; tau++)
#pragma unroll
      for (int pi = 0; pi < 2; pi++)
#pragma unroll
        for (int g = 0; g < G; g++) {
          const int i0 = 2 * pi, i1 = 2 * pi + 1;
          const float P0 = pr[tau][i0] * vs[tau][i0][g], P1 = pr[tau][i1] * vs[tau][i1][g];
          const uint32_t ph = pack_bf16(P0, P1);
          const float h0 = bf_lo(ph), h1 = bf_hi(ph);
          const uint32_t pl = pack_bf16(P0 - h0, P1 - h1);
          pk[tau][pi][g][0] = ph;
          pk[tau][pi][g][1] = pl;
          // the offset uses the fp32 P: hi + lo differs from it by the
          // rounding of lo (~2^-17 P), which times MAG + C0 stays far
          // below the output's own rounding
          float cc = corr[g];
          cc = fmaf(pr[tau][i0], fmaf(C0, vs[tau][i0][g], vb[tau][i0][g]), cc);
          cc = fmaf(pr[tau][i1], fmaf(C0, vs[tau][i1][g], vb[tau][i1][g]), cc);
          cc = fmaf(-(MAG + C0), P0 + P1, cc);
          corr[g] = cc;
        }

    // ---- O^T[dim][head] += V^T . P, one 32-token sub-block per K step
    sfor<2>([&](auto s_) {
      constexpr int s = decltype(s_)::value;
      u32x4_t bpv[G][2];
      sfor<4>([&](auto r_) {
        constexpr int r = decltype(r_)::value;
        constexpr int c = 2 * s + (r >> 1), ts = c / PP, ps = c % PP, pi = r & 1;
#pragma unroll
        for (int g = 0; g < G; g++) {
          bpv[g][0][r] = row_read<ps * HP>(pk[ts][pi][g][0]);
          bpv[g][1][r] = row_read<ps * HP>(pk[ts][pi][g][1]);
        }
      });
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const int g = t / (NT / G);
        if constexpr (BITS == 4) {
          const u32x4_t av = nib_magic(vw[s][t], mg);
          oacc[t] = mfma(av, bpv[g][0], oacc[t]);
          oacc[t] = mfma(av, bpv[g][1], oacc[t]);
        } else {
          u32x4_t lo, hi;
          byte_magic(vw[s][2 * t], vw[s][2 * t + 1], mg, lo, hi);
          oacc[t] = mfma(lo, bpv[g][0], oacc[t]);
          oacc[t] = mfma(lo, bpv[g][1], oacc[t]);
          oacc[t] = mfma(hi, bpv[g][0], oacc[t]);
          oacc[t] = mfma(hi, bpv[g][1], oacc[t]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    });
  };

  // ---- end of a segment: the output itself, or this wave's partial
  auto finalize = [&]() __attribute__((always_inline)) {
    if constexpr (MODE == kModeScores) return;  // the scores are written per step
    float lsum = l_run, csum[G];
#pragma unroll
    for (int g = 0; g < G; g++) csum[g] = corr[g];
    sfor<PP>([&](auto k_) {
      constexpr int kk = decltype(k_)::value;
      if constexpr (kk > 0 && (kk & (kk - 1)) == 0) {  // offsets HP, 2 HP, ... below 16
        lsum += row_readf<kk * HP>(lsum);
#pragma unroll
        for (int g = 0; g < G; g++) csum[g] += row_readf<kk * HP>(csum[g]);
      }
    });
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
#pragma unroll
    for (int g = 0; g < G; g++) {
      csum[g] += __shfl_xor(csum[g], 16);
      csum[g] += __shfl_xor(csum[g], 32);
    }
    const int nst = (seg_len + 63) >> 6;
    const bool whole = seg_t == 0 && seg_take == nst;
    // the pair's units start at unit pa; its partials take the slots of the
    // waves wa..wb that cover it
    const int pa = seg_pa;
    const int wa = pa / cper, wb = (pa + nst - 1) / cper;
    const int64_t pair = static_cast<int64_t>(seg_seq) * HG + seg_j;
    if (seg_t + seg_take == nst && lane == 0)
      reinterpret_cast<int32_t*>(a.ws_ml + a.ws_hdr)[pair] = wb - wa + 1;
    const int64_t hq0 = static_cast<int64_t>(seg_j / n_hg) * rep + (seg_j % n_hg) * HP;
    if (n < nh) {
      if (whole) {
        // (the stored weights are final: no normalisation)
        const float inv = MODE == kModeWeights ? 1.0f : lsum > 0.0f ? 1.0f / lsum : 0.0f;
        uint16_t* o = a.out + seg_seq * a.o_ss + (hq0 + n) * a.o_sh + 4 * lg;
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const float cg = csum[t / (NT / G)];
          u32x2_t v;
          v[0] = out_el<DT>((oacc[t][0] + cg) * inv) | (out_el<DT>((oacc[t][1] + cg) * inv) << 16);
          v[1] = out_el<DT>((oacc[t][2] + cg) * inv) | (out_el<DT>((oacc[t][3] + cg) * inv) << 16);
          *reinterpret_cast<u32x2_t*>(o + 16 * t) = v;
        }
      } else if (merge_here) {
        // device-coherent stores (written through to the level every XCD
        // reads), for the wave that merges the pair.  8 bytes a store: the
        // row's 8-byte words are ordered (t, half e, lane group lg) so that
        // each store instruction writes 32 contiguous bytes of a row (word
        // 8 t + 4 e + lg holds dims 16 t + 4 lg + 2 e, + 1)
        const int64_t slot = pair * a.max_parts + (w - wa);
        uint64_t* o = reinterpret_cast<uint64_t*>(a.ws_o + (slot * HP + n) * D) + lg;
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const float cg = csum[t / (NT / G)];
          __hip_atomic_store(o + 8 * t, pack_f2(oacc[t][0] + cg, oacc[t][1] + cg),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(o + 8 * t + 4, pack_f2(oacc[t][2] + cg, oacc[t][3] + cg),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (lg == 0)
          __hip_atomic_store(reinterpret_cast<uint64_t*>(a.ws_ml) + slot * HP + n,
                             pack_f2(m_run, lsum), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        const int64_t slot = pair * a.max_parts + (w - wa);
        float* o = a.ws_o + (slot * HP + n) * D + 4 * lg;
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const float cg = csum[t / (NT / G)];
          *reinterpret_cast<f32x4_t*>(o + 16 * t) =
              f32x4_t{oacc[t][0] + cg, oacc[t][1] + cg, oacc[t][2] + cg, oacc[t][3] + cg};
        }
        if (lg == 0) {
          // weights mode: plain sums, merged with max 0 and the pair's
          // first partial carrying the sum 1
          a.ws_ml[(slot * HP + n) * 2] = MODE == kModeWeights ? 0.0f : m_run;
          a.ws_ml[(slot * HP + n) * 2 + 1] = MODE == kModeWeights ? (w == wa ? 1.0f : 0.0f) : lsum;
        }
      }
    }
    if (merge_here && !whole) {
      if (pend_pair0 < 0) {
        pend_pair0 = static_cast<int>(pair);
        pend_k0 = wb - wa + 1;
      } else {
        pend_pair1 = static_cast<int>(pair);
        pend_k1 = wb - wa + 1;
      }
    }
    // the next segment's first step refreshes the max from -inf, which
    // scales the accumulators, l_run and corr by zero; the weights mode has
    // no max, so it clears them here
    m_run = -INFINITY;
    if constexpr (MODE == kModeWeights) {
#pragma unroll
      for (int t = 0; t < NT; t++) oacc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < G; g++) corr[g] = 0.0f;
    }
  };

  // ---- the range: unit ui computes while unit ui + 1 loads, and the next
  // segment's queries load at the start of each segment.  Prefetches are
  // unconditional, clamped to the last unit: a conditional load makes the
  // compiler merge the buffer registers at the join, which waits for the
  // loads right after issuing them.  The loop over unit pairs has its only
  // exit at its end: an exit between the two halves gives the wait-count
  // analysis a path on which the second half's loads were never issued, and
  // it then waits for every load in flight before issuing the next ones.
  auto unit = [&](int ui, const Buf& cur, Buf& nxt, auto prefetch) __attribute__((always_inline)) {
    if constexpr (decltype(prefetch)::value) {
      load_step(min(ui + 1, nunits - 1), nxt);
      __builtin_amdgcn_sched_barrier(0);  // issue the loads before any compute
    }
    if constexpr (WPG > 1) {
      if (partner >= 0) {
        __hip_atomic_store(&done_of[wv], ui, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const int other = __builtin_amdgcn_readfirstlane(
            __hip_atomic_load(&done_of[partner], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (other > ui) __builtin_amdgcn_s_setprio(1);       // behind: issue first
        else if (other < ui) __builtin_amdgcn_s_setprio(0);  // ahead: yield
      }
    }
    compute_step(seg_t + (ui - seg_first), cur, cur.vw);
    if (ui == seg_first + seg_take - 1) {  // last unit of the segment
      finalize();
      if (k + 1 < nseg) {
        k++;
        setup_segment(k, qpre);
        if constexpr (MODE != kModeWeights) load_q(min(k + 1, nseg - 1), qpre);
      }
    }
  };
  if constexpr (C::kPrefetch) {
    // pairs of units, the loop's only exit at its end; an odd last unit
    // follows on its own
    int ui = 0;
    for (; ui + 1 < nunits; ui += 2) {
      unit(ui, bufA, bufB, std::true_type{});
      unit(ui + 1, bufB, bufA, std::true_type{});
    }
    if (ui < nunits) unit(ui, bufA, bufB, std::false_type{});
  } else if constexpr (C::kPrefetchK) {
    // unit ui: its value words, then unit ui + 1's key words (clamped,
    // unconditional), issued before it computes; the value words' latency
    // hides behind the scores
    auto unit_k = [&](int ui, const Buf& cur, Buf& nxt) __attribute__((always_inline)) {
      load_v(ui, vcur);
      load_k(min(ui + 1, nunits - 1), nxt);
      __builtin_amdgcn_sched_barrier(0);
      compute_step(seg_t + (ui - seg_first), cur, vcur);
      if (ui == seg_first + seg_take - 1) {
        finalize();
        if (k + 1 < nseg) {
          k++;
          setup_segment(k, qpre);
          if constexpr (MODE != kModeWeights) load_q(min(k + 1, nseg - 1), qpre);
        }
      }
    };
    int ui = 0;
    for (; ui + 1 < nunits; ui += 2) {
      unit_k(ui, bufA, bufB);
      unit_k(ui + 1, bufB, bufA);
    }
    if (ui < nunits) unit_k(ui, bufA, bufB);
  } else {
    for (int ui = 0;; ui++) {
      compute_step(seg_t + (ui - seg_first), bufA, bufA.vw);
      if (ui == seg_first + seg_take - 1) {
        finalize();
        if (ui + 1 == nunits) break;
        k++;
        setup_segment(k, qpre);
        if constexpr (MODE != kModeWeights) load_q(min(k + 1, nseg - 1), qpre);
      }
      load_step(ui + 1, bufA);
    }
  }
  if (pend_pair0 >= 0) {
    // Counted in at the range's end, where no loads are left to wait for:
    // this wave's partial stores are complete first.  The wave that counts
    // a pair's last partial zeroes the counter for the next launch and
    // merges the pair.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // both counts in one round trip, then both merges' first loads together
    uint32_t b0 = 0, b1 = 0;
    if (lane == 0) {
      b0 = __hip_atomic_fetch_add(a.counters + pend_pair0, 1u, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
      if (pend_pair1 >= 0)
        b1 = __hip_atomic_fetch_add(a.counters + pend_pair1, 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    }
    const bool last0 = __builtin_amdgcn_readfirstlane(b0) == static_cast<uint32_t>(pend_k0 - 1);
    const bool last1 =
        pend_pair1 >= 0 && __builtin_amdgcn_readfirstlane(b1) == static_cast<uint32_t>(pend_k1 - 1);
    if (lane == 0) {
      if (last0) __hip_atomic_store(a.counters + pend_pair0, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (last1) __hip_atomic_store(a.counters + pend_pair1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (last0 && last1) {
      const int pr[2] = {pend_pair0, pend_pair1}, kk[2] = {pend_k0, pend_k1};
      qdecode_merge_pairs<HP, D, DT, 2>(a, pr, kk, lane);
    } else if (last0 || last1) {
      const int pr[1] = {last0 ? pend_pair0 : pend_pair1}, kk[1] = {last0 ? pend_k0 : pend_k1};
      qdecode_merge_pairs<HP, D, DT, 1>(a, pr, kk, lane);
    }
  }
}

// Merge of the partials of (sequence, head pair)s that several waves
// share (sdpa_vector.h:320-394).  Block = one (sequence, pair), thread = 4
// dims of one head.  The pair's partial count, its length and its first NF
// partials load together (the partial slots past the count hold stale
// data, which the merge masks), so a pair of up to NF partials costs one
// round trip to memory.  With REST the rest of a pair's first kMaxParts
// partials (only those below the count) then load together, a second round
// trip; without it they load 4 at a time (the host picks REST when launches
// average more than 4 waves per pair).  Partials past kMaxParts (long
// sequences) load 4 a round trip.  (Loading 16 with the count measured
// slower where most pairs have few partials, the stale slots costing
// traffic; loading all 32 with the count for config 2's 32 partials a pair
// took the merge from 4.7 to 10.4 us.)
template <int HP, int NF, bool REST, int DT>
__global__ void __launch_bounds__(512) qdecode_combine_kernel(DecodeArgs a, int D) {
  constexpr int kQuad = 4;
  const int rep = a.rep, n_hg = (rep + HP - 1) / HP, HG = a.Hkv * n_hg;
  const int P = blockIdx.x, seq = P / HG, j = P % HG;
  const int len = a.seq_lens ? a.seq_lens[seq] : a.max_len;
  // (clamped: a count the decode kernel did not write stays within the slots)
  const int K = min(reinterpret_cast<const int32_t*>(a.ws_ml + a.ws_hdr)[P], a.max_parts);
  const int64_t hq0 = static_cast<int64_t>(j / n_hg) * rep + (j % n_hg) * HP;
  const int nh = min(HP, rep - (j % n_hg) * HP);
  const int64_t slot0 = static_cast<int64_t>(P) * a.max_parts;
  const int r = threadIdx.x / (D / 4), d = 4 * (threadIdx.x % (D / 4));
  if (r >= HP) return;
  float M = -INFINITY, L = 0.0f, o[4] = {0.f, 0.f, 0.f, 0.f};
  auto merge = [&](int k0, auto N_, const f32x2_t* ml, const f32x4_t* oo) __attribute__((always_inline)) {
    constexpr int N = decltype(N_)::value;
    float mlm[N], mll[N], ov[N][4];
#pragma unroll
    for (int q = 0; q < N; q++) {
      mlm[q] = ml[q][0];
      mll[q] = ml[q][1];
#pragma unroll
      for (int e = 0; e < 4; e++) ov[q][e] = oo[q][e];
    }
    qmerge_step<N, 4>(M, L, o, k0, K, mlm, mll, ov);
  };
  // slots k0 .. k0 + N - 1 (clamped to the last live one), loaded together
  auto load = [&](int k0, auto N_, f32x2_t* ml, f32x4_t* oo) __attribute__((always_inline)) {
    constexpr int N = decltype(N_)::value;
#pragma unroll
    for (int q = 0; q < N; q++) {
      const int64_t slot = (slot0 + min(k0 + q, max(K - 1, 0))) * HP + r;
      ml[q] = *reinterpret_cast<const f32x2_t*>(a.ws_ml + slot * 2);
      oo[q] = *reinterpret_cast<const f32x4_t*>(a.ws_o + slot * D + d);
    }
  };
  {
    f32x2_t ml[NF];
    f32x4_t oo[NF];
#pragma unroll
    for (int q = 0; q < NF; q++) {  // unclamped: issued beside the count's load
      const int64_t slot = (slot0 + q) * HP + r;
      ml[q] = *reinterpret_cast<const f32x2_t*>(a.ws_ml + slot * 2);
      oo[q] = *reinterpret_cast<const f32x4_t*>(a.ws_o + slot * D + d);
    }
    if (len == 0 || K <= 1 || r >= nh) return;  // written by the decode kernel itself
    merge(0, std::integral_constant<int, NF>{}, ml, oo);
  }
  int k0 = NF;
  if (REST && NF < kMaxParts && K > NF) {
    constexpr int kRest = kMaxParts - NF > 0 ? kMaxParts - NF : 1;
    f32x2_t ml[kRest];
    f32x4_t oo[kRest];
#pragma unroll
    for (int q = 0; q < kRest; q++) {
      if (NF + q < K) {
        const int64_t slot = (slot0 + NF + q) * HP + r;
        ml[q] = *reinterpret_cast<const f32x2_t*>(a.ws_ml + slot * 2);
        oo[q] = *reinterpret_cast<const f32x4_t*>(a.ws_o + slot * D + d);
      } else {
        ml[q] = f32x2_t{-INFINITY, 0.0f};
        oo[q] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
    merge(NF, std::integral_constant<int, kRest>{}, ml, oo);
    k0 = kMaxParts;
  }
  for (; k0 < K; k0 += kQuad) {
    f32x2_t ml[kQuad];
    f32x4_t oo[kQuad];
    load(k0, std::integral_constant<int, kQuad>{}, ml, oo);
    merge(k0, std::integral_constant<int, kQuad>{}, ml, oo);
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  u32x2_t v;
  v[0] = out_el<DT>(o[0] * inv) | (out_el<DT>(o[1] * inv) << 16);
  v[1] = out_el<DT>(o[2] * inv) | (out_el<DT>(o[3] * inv) << 16);
  *reinterpret_cast<u32x2_t*>(a.out + seq * a.o_ss + (hq0 + r) * a.o_sh + d) = v;
}

static int heads_per_part(int rep) { return rep <= 4 ? 4 : 8; }

int qdecode_head_groups(int rep) { return (rep + heads_per_part(rep) - 1) / heads_per_part(rep); }

bool qdecode_supported(int dtype, int bits, int D, int block_size, int rep, int group) {
  return (dtype == kBF16 || dtype == kF16) && (bits == 4 || bits == 8) &&
         (D == 64 || D == 128 || D == 256) && block_size % 32 == 0 && rep >= 1 && rep <= 16 &&
         (group == 64 || (group == 128 && D >= 128));
}

int qdecode_waves(int n_seqs, int Hkv, int rep, int max_len, int want) {
  // cost units (steps + kSegCost per pair), at most
  const int64_t units = static_cast<int64_t>(n_seqs) * Hkv * qdecode_head_groups(rep) *
                        ((static_cast<int64_t>(max_len) + 63) / 64 + kSegCost);
  const int64_t need = (units + kMaxRange - 1) / kMaxRange;  // ranges of at most kMaxRange units
  // one round of resident waves (2 per SIMD x 4 SIMDs x 256 CUs), down to
  // 2 units per wave for small launches (8 x 4096 tokens: 2048 waves ran
  // 13% faster than 1040 at 4 units each)
  int64_t waves = want > 0 ? want : std::min<int64_t>(2048, (units + 1) / 2);
  waves = std::max<int64_t>({waves, need, 1});
  return static_cast<int>(waves);
}

// Partials per (sequence, head pair) a launch allows: kMaxParts, or as many
// as keep every wave's range within kMaxRange units for the longest
// sequence.
int qdecode_max_parts(int max_len) {
  const int max_nst = (std::max(max_len, 1) + 63) / 64;
  return std::max(kMaxParts, (max_nst + kMaxRange - 1) / kMaxRange + 2);
}

size_t qdecode_workspace_floats(int n_seqs, int Hkv, int rep, int D, int max_len) {
  const int hp = heads_per_part(rep);
  const size_t pairs = static_cast<size_t>(n_seqs) * Hkv * qdecode_head_groups(rep);
  // + one partial count (int32) per pair
  return pairs * qdecode_max_parts(max_len) * hp * (D + 2) + pairs;
}

int qdecode_max_seqs() { return kMaxSeqs; }

// ---- scratch of the no-allocation decode entry point (vkv_paged_sdpa_noalloc)
// Its split-K partials live in this fixed array instead of a workspace the
// library allocates, for callers that cannot allocate device memory.  Each
// device the library runs on holds its own copy from module load until the
// process ends.  Every call on a device shares that device's copy: calls
// that overlap on one device race.  The partials need no clearing: each
// launch writes every slot it later reads (the partial count of a pair is
// written by the wave that ends it; empty sequences are never merged).
constexpr size_t kScratchBytes = size_t{64} << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

size_t decode_scratch_bytes() { return kScratchBytes; }

float* decode_scratch(size_t floats) {
  if (floats > kScratchBytes / sizeof(float))
    throw Error("the call needs " + std::to_string(floats * sizeof(float)) +
                " bytes of split-K scratch; the no-allocation entry point holds " +
                std::to_string(kScratchBytes) + " (fewer sequences per call fit)");
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  VKV_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) throw Error("device index out of range for the scratch table");
  std::lock_guard<std::mutex> g(mu);
  if (!addr[dev]) {
    // the host-side name of a __device__ array is not its device address
    void* p = nullptr;
    VKV_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) throw Error("hipGetSymbolAddress(scratch) returned NULL");
    addr[dev] = p;
  }
  return static_cast<float*>(addr[dev]);
}

// Longest sequence the decode kernel takes (its cost units stay in int32
// for a launch of kMaxSeqs sequences).
int qdecode_max_len() { return 1 << 24; }

template <int BITS, int D, int HP, int DT>
static void launch_hp(const DecodeArgs& a0, bool ref, hipStream_t st) {
  constexpr int wpg = qd_waves<D>();
  const dim3 grid((a0.n_waves + wpg - 1) / wpg), block(64 * wpg);
  const int pairs = a0.n_seqs * a0.Hkv * qdecode_head_groups(a0.rep);
  const bool rest = a0.n_waves > 4 * pairs;  // more than kFirst partials per pair on average
  // The partials merge inside the fused launch (each wave counts its
  // partials in at its range's end; the last of a pair merges it) where
  // pairs average at most 4 partials, at most 128 dims; longer merges
  // (config 2: 32 partials a pair) and 256 dims keep the merge launch.
  DecodeArgs a = a0;
  if (ref || rest || D > 128) a.counters = nullptr;
  if (ref) VKV_CHECK(a.group == 64, "the matrix-core reference path takes group 64");
  if constexpr (DT == kBF16) {
    if (ref) {
      // the reference-arithmetic path: bf16 score rows, the reference
      // softmax over them in place, then P.V from the stored weights
      hipLaunchKernelGGL((qdecode_kernel<BITS, D, HP, kModeScores, DT>), grid, block, 0, st, a);
      VKV_HIP(hipGetLastError());
      launch_ref_softmax_bf16(a.sc, static_cast<int64_t>(a.n_seqs) * a.Hq, a.sc_stride,
                              a.seq_lens, a.max_len, a.Hq, st);
      const TimedLaunch tl = timing_prepare(kTimeDecode);
      hipExtLaunchKernelGGL((qdecode_kernel<BITS, D, HP, kModeWeights, DT>), grid, block, 0, st,
                            tl.start, tl.stop, 0, a);
      VKV_HIP(hipGetLastError());
      timing_commit(tl);
    }
  } else {
    if (ref) throw Error("the matrix-core reference path takes bf16 caches");
  }
  if (!ref) {
    const TimedLaunch tl = timing_prepare(kTimeDecode);
    if (a.group == 128) {
      if constexpr (D >= 128) {
        VKV_CHECK(a.new_k == nullptr, "a group-128 decode takes no decode token");
        hipExtLaunchKernelGGL((qdecode_kernel<BITS, D, HP, kModeFusedG128, DT>), grid, block, 0,
                              st, tl.start, tl.stop, 0, a);
      } else {
        throw Error("group 128 needs head dims of at least 128");
      }
    } else {
      VKV_CHECK(a.group == 64, "the matrix-core decode takes groups of 64 or 128");
      hipExtLaunchKernelGGL((qdecode_kernel<BITS, D, HP, kModeFused, DT>), grid, block, 0, st,
                            tl.start, tl.stop, 0, a);
    }
    VKV_HIP(hipGetLastError());
    timing_commit(tl);
  }
  if (a.counters) return;
  const dim3 cb(HP == 4 ? D : 2 * D);
  if (rest)
    hipLaunchKernelGGL((qdecode_combine_kernel<HP, 4, true, DT>), dim3(pairs), cb, 0, st, a, D);
  else
    hipLaunchKernelGGL((qdecode_combine_kernel<HP, 4, false, DT>), dim3(pairs), cb, 0, st, a, D);
  VKV_HIP(hipGetLastError());
}

template <int BITS, int D, int DT>
static void launch_d(const DecodeArgs& a, bool ref, hipStream_t st) {
  if (heads_per_part(a.rep) == 4) launch_hp<BITS, D, 4, DT>(a, ref, st);
  else launch_hp<BITS, D, 8, DT>(a, ref, st);
}

template <int DT>
static void launch_dt(const DecodeArgs& a, int bits, int D, bool ref, hipStream_t st) {
  if (bits == 4) {
    if (D == 64) launch_d<4, 64, DT>(a, ref, st);
    else if (D == 128) launch_d<4, 128, DT>(a, ref, st);
    else launch_d<4, 256, DT>(a, ref, st);
  } else {
    if (D == 64) launch_d<8, 64, DT>(a, ref, st);
    else if (D == 128) launch_d<8, 128, DT>(a, ref, st);
    else launch_d<8, 256, DT>(a, ref, st);
  }
}

void launch_qdecode(const DecodeArgs& a0, int bits, int D, hipStream_t st, bool ref) {
  VKV_CHECK(a0.dtype == kBF16 || a0.dtype == kF16, "the matrix-core decode takes bf16 or f16 caches");
  // at most kMaxSeqs sequences per launch
  for (int s0 = 0; s0 < a0.n_seqs; s0 += kMaxSeqs) {
    DecodeArgs a = a0;
    a.n_seqs = std::min(kMaxSeqs, a0.n_seqs - s0);
    a.n_waves = qdecode_waves(a.n_seqs, a.Hkv, a.rep, a.max_len, a0.n_waves);
    a.max_parts = qdecode_max_parts(a.max_len);
    const size_t slots = static_cast<size_t>(a.n_seqs) * a.Hkv * qdecode_head_groups(a.rep) * a.max_parts;
    a.ws_o = a0.ws;
    a.ws_ml = a0.ws + slots * heads_per_part(a.rep) * D;
    a.ws_hdr = static_cast<int32_t>(slots * heads_per_part(a.rep) * 2);
    a.q += s0 * a0.q_ss;
    a.out += s0 * a0.o_ss;
    a.table += static_cast<int64_t>(s0) * a0.table_stride;
    if (a.seq_lens) a.seq_lens += s0;
    if (a.new_k) {
      a.new_k += s0 * a0.nk_ss;
      a.new_v += s0 * a0.nv_ss;
    }
    if (a.dtype == kF16) launch_dt<kF16>(a, bits, D, ref, st);
    else launch_dt<kBF16>(a, bits, D, ref, st);
  }
}

}  // namespace vkv
