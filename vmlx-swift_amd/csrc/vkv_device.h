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

}  // namespace vkv
