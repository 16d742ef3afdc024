// vkv_device.h -- device-side helpers shared by the HIP kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace vkv {

enum DType { kF32 = 0, kF16 = 1, kBF16 = 2 };

// Bit-exact IEEE round-to-nearest-even conversions.  bf16 is done on the
// integer pattern so the result never depends on the compiler's rounding
// mode; f16 uses the hardware cvt (v_cvt_f16_f32 rounds to nearest even).
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

template <int DT> struct Elem;
template <> struct Elem<kF32> {
  using T = float;
  static constexpr int kBytes = 4;
  __device__ __forceinline__ static float load(const T* p) { return *p; }
  __device__ __forceinline__ static T from_f32(float f) { return f; }
  __device__ __forceinline__ static float to_f32(T v) { return v; }
  // Largest finite value (Limits<T>::max) and lowest (finfo.min).
  static constexpr float kMax = 3.402823466e38f;
};
template <> struct Elem<kF16> {
  using T = uint16_t;
  static constexpr int kBytes = 2;
  __device__ __forceinline__ static float load(const T* p) { return f16_to_f32(*p); }
  __device__ __forceinline__ static T from_f32(float f) { return f32_to_f16(f); }
  __device__ __forceinline__ static float to_f32(T v) { return f16_to_f32(v); }
  static constexpr float kMax = 65504.0f;
};
template <> struct Elem<kBF16> {
  using T = uint16_t;
  static constexpr int kBytes = 2;
  __device__ __forceinline__ static float load(const T* p) { return bf16_to_f32(*p); }
  __device__ __forceinline__ static T from_f32(float f) { return f32_to_bf16(f); }
  __device__ __forceinline__ static float to_f32(T v) { return bf16_to_f32(v); }
  static constexpr float kMax = 3.38953139e38f;
};

template <int DT>
__device__ __forceinline__ float round_to(float f) {
  return Elem<DT>::to_f32(Elem<DT>::from_f32(f));
}

// Element i of a float array of dtype `dt` (kF32, kF16 or kBF16) as fp32,
// rounded to the dtype DT of the attention (the reference kernels read
// masks and sinks as the query dtype T, sdpa_vector.h:15-38).
__device__ __forceinline__ float load_f32(const void* p, int dt, int64_t i) {
  if (dt == kF16) return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
  if (dt == kBF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  return static_cast<const float*>(p)[i];
}
template <int DT>
__device__ __forceinline__ float load_as(const void* p, int dt, int64_t i) {
  const float v = load_f32(p, dt, i);
  return dt == DT ? v : round_to<DT>(v);
}

// ---------------------------------------------------------------------------
// Affine paged chunk format (block_size % 32 == 0, head_dim % 32 == 0).
// One (block, kv head) chunk holds K codes, V codes, then the scale/bias
// area.  The word orders are chosen so that each lane of the decode kernel
// reads its MFMA operands with one contiguous 16-byte load:
//  * K codes are token-major (a row of D*bits/32 words per token).  Within a
//    row, original word w (the reference's little-endian packing: element i
//    of the row lives in word i*bits/32) is stored at position
//      4-bit: kg*(D/32) + s            with s = w / 4, kg = w % 4
//      8-bit: (kg*(D/32) + s)*2 + h    with q = w / 2, s = q / 4, kg = q % 4,
//                                      h = w % 2
//    i.e. the words one MFMA lane group (kg) needs for every 32-dim K step
//    (s) are adjacent.
//  * V codes are dim-major per 32-token sub-block: the 8 tokens
//    8*kg .. 8*kg+7 of dim d = 16*mt + m share one word (4-bit; two words
//    for 8-bit) at
//      4-bit: (kg*16 + m)*(D/16) + mt
//      8-bit: ((kg*16 + m)*(D/16) + mt)*2 + (q/4)
//    token 8*kg + q sits at bit bits*(q % (32/bits)) of its word.
//  * scale/bias: per token 4*G values (2*G when keys-only) of the element
//    dtype: [K: (scale, bias) x G][V: (scale, bias) x G].
__device__ __forceinline__ int64_t qk_word_off(int64_t t, int w, int D, int bits) {
  const int row_words = D * bits / 32;
  int idx;
  if (bits == 4) {
    idx = (w & 3) * (D / 32) + (w >> 2);
  } else {
    const int q = w >> 1;
    idx = ((q & 3) * (D / 32) + (q >> 2)) * 2 + (w & 1);
  }
  return (t * row_words + idx) * 4;
}

__device__ __forceinline__ int64_t qv_word_off(int64_t t, int d, int D, int bits, int* shift) {
  const int64_t sb = t >> 5;
  const int tt = static_cast<int>(t & 31);
  const int kg = tt >> 3, q = tt & 7, m = d & 15, mt = d >> 4, NT = D >> 4;
  int64_t idx = sb * static_cast<int64_t>(D) * bits;
  if (bits == 4) {
    idx += (kg * 16 + m) * NT + mt;
    *shift = 4 * q;
  } else {
    idx += ((kg * 16 + m) * NT + mt) * 2 + (q >> 2);
    *shift = 8 * (q & 3);
  }
  return idx * 4;
}

__device__ __forceinline__ int64_t qsb_index(int64_t t, int which, int g, int sel, int G,
                                             bool keys_only) {
  return t * (keys_only ? 2 * G : 4 * G) + which * 2 * G + g * 2 + sel;
}

// Two floats as one 64-bit word (first in the low half), for the
// device-coherent 64-bit stores of split-K partials.
__device__ __forceinline__ uint64_t pack_f2(float lo, float hi) {
  return static_cast<uint64_t>(__float_as_uint(lo)) | (static_cast<uint64_t>(__float_as_uint(hi)) << 32);
}

__device__ __forceinline__ float wave_max(float v, int width) {
  for (int o = width / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, width));
  return v;
}
__device__ __forceinline__ float wave_min(float v, int width) {
  for (int o = width / 2; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, width));
  return v;
}
__device__ __forceinline__ float wave_sum(float v, int width) {
  for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, width);
  return v;
}

// The reference's affine quantization of a group (quantized.h:2422-2458),
// 8 values of the group a lane, GROUP / 8 neighbouring lanes a group (every
// lane of the team calls it), operation for operation in fp32 with IEEE
// division and round-half-away-from-zero:
//   running min starts at Limits<T>::max, running max at 0 (:2422-2431);
//   scale = max((max - min) / n_bins, 1e-7), negated when max is the edge,
//   q0 = round(edge / scale), scale = edge / q0, bias = edge unless q0 == 0
//   (:2436-2443);
//   code = min(round((w - bias) / scale), n_bins) with the unrounded scale
//   (:2458); the caller stores scale and bias rounded to T (:2447-2450).
template <int DT, int BITS, int GROUP>
__device__ __forceinline__ void affine_quantize8(const float (&v)[8], uint32_t (&code)[8],
                                                 float& scale_out, float& bias_out) {
  constexpr int TEAM = GROUP / 8;
  constexpr float n_bins = static_cast<float>((1 << BITS) - 1);
  float w_min = Elem<DT>::kMax, w_max = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    w_min = fminf(w_min, v[e]);
    w_max = fmaxf(w_max, v[e]);
  }
  w_min = wave_min(w_min, TEAM);
  w_max = wave_max(w_max, TEAM);
  float scale = fmaxf((w_max - w_min) / n_bins, 1e-7f);
  const bool side = fabsf(w_min) > fabsf(w_max);
  scale = side ? scale : -scale;
  const float edge = side ? w_min : w_max;
  const float q0 = roundf(edge / scale);
  const bool at_zero = q0 == 0.0f;
  scale = at_zero ? scale : edge / q0;
  const float bias = at_zero ? 0.0f : edge;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float x = fminf(roundf((v[e] - bias) / scale), n_bins);
    code[e] = x > 0.0f ? static_cast<uint32_t>(x) : 0u;
  }
  scale_out = scale;
  bias_out = bias;
}

}  // namespace vkv
