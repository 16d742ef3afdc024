// vkv_tq.hip -- the TurboQuant KV codec on the device
// (Libraries/MLXLMCommon/TurboQuant/TQEncoder.swift, TQHadamard.swift,
// TQCodebook.swift, TQQJL.swift, TQBitPack.swift).
//
// Encode (keys or values): per vector, the norm in the input dtype T, the
// unit vector in T, the randomized blockwise Hadamard rotation (f32), the
// Lloyd-Max code of every coordinate and, for keys, the residual's norm and
// the signs of its projection through the QJL matrix; codes and signs are
// packed into the reference's flat u32 words (value e of the tensor in word
// e / (32 / bits) at bit (e % (32 / bits)) * bits).  Decode: codebook
// lookup, the QJL correction sqrt(pi/2)/d * |r| * (signs . S) for keys, the
// inverse rotation, times the stored norm, to f16, written straight into the
// cache's unified buffer (f16 or f32) at the vector's token position.
//
// A workgroup of 256 threads takes tiles of 32 vectors through LDS.  The
// two matrix products run as f32 fused multiply-add chains in index order
// (one output per thread and row, the matrix read coalesced from L2), the
// row sums in double; the same orders are what the CPU restatement fixes,
// so the codes, signs, norms and decoded values are bit-exact with it.
// Contraction is off in this file: every other product and sum rounds as
// the reference writes it.
#include "vkv_device.h"
#include "vkv_internal.h"

#pragma clang fp contract(off)

namespace vkv {
namespace {

constexpr int kRows = kTqTileRows;
constexpr int kThreads = 256;

// f16 of an f32 value that is first rounded to f32: the barrier keeps the
// compiler from folding the product or sum that made v into a mixed
// precision fma that rounds once, straight to f16 (v_fma_mix*).
__device__ __forceinline__ uint16_t f16_of(float v) {
  asm volatile("" : "+v"(v));
  return f32_to_f16(v);
}

__device__ __forceinline__ float round_dt(float v, int dt) {
  if (dt == kF16) return f16_to_f32(f16_of(v));
  if (dt == kBF16) return bf16_to_f32(f32_to_bf16(v));
  return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// The blockwise butterfly of TQHadamard.hadamardTransform over a tile of
// `rows` vectors held in LDS (row stride D): every block runs its stages
// (a + b, a - b) on pairs (g 2h + j, g 2h + h + j), then scales by its
// f32 1 / sqrt(n).
__device__ void hadamard_tile(float* y, int rows, int D, const TqBlocks& bl) {
  const int tid = threadIdx.x;
  for (int b = 0; b < bl.n; ++b) {
    const int n = bl.size[b], off = bl.off[b], half = n >> 1;
    for (int h = 1; h < n; h <<= 1) {
      __syncthreads();
      for (int p = tid; p < rows * half; p += kThreads) {
        const int r = p / half, q = p - r * half;
        const int g = q / h, j = q - g * h;
        float* v = y + r * D + off + g * 2 * h + j;
        const float a = v[0], c = v[h];
        v[0] = a + c;
        v[h] = a - c;
      }
    }
    __syncthreads();
    const float s = bl.scale[b];
    for (int p = tid; p < rows * n; p += kThreads) {
      const int r = p / n, i = p - r * n;
      y[r * D + off + i] = y[r * D + off + i] * s;
    }
  }
  __syncthreads();
}

// Packs the tile's values (u8, tile element k = flat element e0 + k) into
// the flat words of `bits` each.  Words wholly inside the tile are stored;
// the (at most two) words it shares with a neighbouring tile are OR-ed into
// the zeroed output.
__device__ void pack_tile(const uint8_t* vals, int64_t e0, int64_t e1, int64_t total, int bits,
                          uint32_t* out) {
  const int vpw = 32 / bits;
  const int64_t w0 = e0 / vpw, w1 = (e1 - 1) / vpw;
  for (int64_t w = w0 + threadIdx.x; w <= w1; w += kThreads) {
    uint32_t word = 0;
    for (int k = 0; k < vpw; ++k) {
      const int64_t e = w * vpw + k;
      if (e >= e0 && e < e1) word |= static_cast<uint32_t>(vals[e - e0]) << (k * bits);
    }
    const int64_t end = (w + 1) * vpw < total ? (w + 1) * vpw : total;
    if (w * vpw >= e0 && end <= e1)
      out[w] = word;
    else if (word)
      atomicOr(out + w, word);
  }
}

__device__ __forceinline__ uint32_t unpack_at(const uint32_t* words, int64_t e, int bits) {
  const int vpw = 32 / bits;
  return (words[e / vpw] >> ((e % vpw) * bits)) & ((1u << bits) - 1u);
}

// acc[r][j] = sum_i a[r][i] * M[i * D + j], an f32 fma chain in i order, for
// the tile's rows, handed to f(r, j, acc) for rows below `rows`; the left
// operand is read as floats, or (SGN) as +-1 from bytes.  DT = D (a power of
// two dividing 256) keeps a register tile of kRows * D / 256 outputs per
// thread; DT = 0 walks (row, j) pairs.  f must not write the operands.
template <int DT, bool SGN, class F>
__device__ void tile_matmul(const float* a, const uint8_t* sa, int rows, int D, const float* M,
                            F&& f) {
  const int tid = threadIdx.x;
  if constexpr (DT > 0) {
    constexpr int G = kThreads / DT;   // row groups
    constexpr int RPT = kRows / G;     // rows per thread
    const int j = tid % DT, g = tid / DT;
    float acc[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) acc[k] = 0.0f;
    for (int i = 0; i < DT; ++i) {
      const float m = M[i * DT + j];
#pragma unroll
      for (int k = 0; k < RPT; ++k) {
        const int r = g + k * G;
        const float x = SGN ? (sa[r * DT + i] ? 1.0f : -1.0f) : a[r * DT + i];
        acc[k] = fmaf(x, m, acc[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int r = g + k * G;
      if (r < rows) f(r, j, acc[k]);
    }
  } else {
    for (int p = tid; p < rows * D; p += kThreads) {
      const int r = p / D, j = p - r * D;
      float acc = 0.0f;
      for (int i = 0; i < D; ++i) {
        const float x = SGN ? (sa[r * D + i] ? 1.0f : -1.0f) : a[r * D + i];
        acc = fmaf(x, M[static_cast<int64_t>(i) * D + j], acc);
      }
      f(r, j, acc);
    }
  }
  __syncthreads();
}

template <int DT>
__global__ void __launch_bounds__(kThreads) tq_encode_kernel(TqEncodeArgs a) {
  extern __shared__ float lds[];
  const int D = DT > 0 ? DT : a.D;
  float* y = lds;                                                   // [kRows][D] f32
  uint8_t* codes = reinterpret_cast<uint8_t*>(y + kRows * D);       // [kRows][D]
  uint8_t* sg = codes + kRows * D;                                  // [kRows][D]
  __shared__ float den_s[kRows];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t rows = static_cast<int64_t>(a.B) * a.H * a.Tc, total = rows * D;
  const bool keys = a.St != nullptr;
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRows; r0 < rows;
       r0 += static_cast<int64_t>(gridDim.x) * kRows) {
    const int nr = static_cast<int>(rows - r0 < kRows ? rows - r0 : kRows);
    // 1. load the tile (rows past the end are zeros)
    for (int e = tid; e < kRows * D; e += kThreads) {
      const int r = e / D, i = e - r * D;
      float v = 0.0f;
      if (r < nr) {
        const int64_t row = r0 + r;
        const int64_t t = row % a.Tc, bh = row / a.Tc, h = bh % a.H, b = bh / a.H;
        v = load_f32(a.x, a.dtype, b * a.sb + h * a.sh + (a.t0 + t) * a.st + i);
      }
      y[e] = v;
    }
    __syncthreads();
    // 2. norm in T: T(sqrt(T(sum T(x_i^2)))), the divisor T(norm + T(1e-8))
    for (int r = wave; r < kRows; r += kThreads / 64) {
      double s = 0.0;
      for (int i = lane; i < D; i += 64) {
        const float v = y[r * D + i];
        s += static_cast<double>(round_dt(v * v, a.dtype));
      }
      s = wave_sum_d(s);
      const float nrm = round_dt(sqrtf(round_dt(static_cast<float>(s), a.dtype)), a.dtype);
      if (lane == 0) {
        den_s[r] = round_dt(nrm + round_dt(1e-8f, a.dtype), a.dtype);
        if (r < nr) a.vec_norms[r0 + r] = f16_of(nrm);
      }
    }
    __syncthreads();
    // 3. unit vector in T, times the rotation signs (f32), rotated
    for (int e = tid; e < kRows * D; e += kThreads) {
      const int r = e / D, i = e - r * D;
      y[e] = round_dt(y[e] / den_s[r], a.dtype) * a.signs[i];
    }
    hadamard_tile(y, kRows, D, a.blocks);
    // 4. codes (boundaries exceeded); keys keep the residual y - level
    for (int e = tid; e < kRows * D; e += kThreads) {
      const float v = y[e];
      int idx = 0;
      for (int k = 0; k < a.nc - 1; ++k) idx += v > a.bounds[k];
      codes[e] = static_cast<uint8_t>(idx);
      if (keys) y[e] = v - a.codebook[idx];
    }
    __syncthreads();
    if (keys) {
      // 5. residual norm: f32(sum f32(r_i^2)) -> sqrt -> f16
      for (int r = wave; r < nr; r += kThreads / 64) {
        double s = 0.0;
        for (int i = lane; i < D; i += 64) {
          const float v = y[r * D + i];
          s += static_cast<double>(v * v);
        }
        s = wave_sum_d(s);
        if (lane == 0) a.res_norms[r0 + r] = f16_of(sqrtf(static_cast<float>(s)));
      }
      // 6. projection through S (S^T as the right operand), signs p >= 0
      tile_matmul<DT, false>(y, nullptr, nr, D, a.St,
                             [&](int r, int j, float v) { sg[r * D + j] = v >= 0.0f; });
    }
    // 7. pack codes and signs into the flat words
    const int64_t e0 = r0 * D, e1 = (r0 + nr) * D;
    pack_tile(codes, e0, e1, total, a.bits, a.indices);
    if (keys) pack_tile(sg, e0, e1, total, 1, a.qjl);
    __syncthreads();
  }
}

template <int DT>
__global__ void __launch_bounds__(kThreads) tq_decode_kernel(TqDecodeArgs a) {
  extern __shared__ float lds[];
  const int D = DT > 0 ? DT : a.D;
  float* z = lds;                                                   // [kRows][D]
  uint8_t* sg = reinterpret_cast<uint8_t*>(z + kRows * D);          // [kRows][D]
  const int tid = threadIdx.x;
  const int64_t rows = static_cast<int64_t>(a.B) * a.H * a.Tc;
  const bool keys = a.S != nullptr;
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRows; r0 < rows;
       r0 += static_cast<int64_t>(gridDim.x) * kRows) {
    const int nr = static_cast<int>(rows - r0 < kRows ? rows - r0 : kRows);
    for (int e = tid; e < kRows * D; e += kThreads) {
      const int r = e / D;
      float v = 0.0f;
      uint8_t s = 0;
      if (r < nr) {
        const int64_t fe = r0 * D + e;
        v = a.codebook[unpack_at(a.indices, fe, a.bits)];
        if (keys) s = static_cast<uint8_t>(unpack_at(a.qjl, fe, 1));
      }
      z[e] = v;
      sg[e] = s;
    }
    __syncthreads();
    if (keys) {
      // z += (sqrt(pi/2) / d * |r|) * (signs . S)
      tile_matmul<DT, true>(nullptr, sg, nr, D, a.S, [&](int r, int j, float v) {
        const float c = a.qs * f16_to_f32(a.res_norms[r0 + r]);
        z[r * D + j] = z[r * D + j] + c * v;
      });
    }
    hadamard_tile(z, kRows, D, a.blocks);
    for (int e = tid; e < kRows * D; e += kThreads) {
      const int r = e / D, i = e - r * D;
      if (r >= nr) continue;
      const int64_t row = r0 + r;
      const float w = z[e] * a.signs[i] * f16_to_f32(a.vec_norms[row]);
      const uint16_t hv = f16_of(w);
      const int64_t t = row % a.Tc, bh = row / a.Tc, h = bh % a.H, b = bh / a.H;
      const int64_t o = b * a.osb + h * a.osh + (a.t0 + t) * a.ost + i;
      if (a.out_dtype == kF16)
        static_cast<uint16_t*>(a.out)[o] = hv;
      else
        static_cast<float*>(a.out)[o] = f16_to_f32(hv);
    }
    __syncthreads();
  }
}

// dst = src converted (4-D strided, element strides, round to nearest even
// when narrowing): the cast of MLX's concatenation and slice assignment.
__global__ void __launch_bounds__(256) cast4d_kernel(const void* src, int sdt, int64_t n0,
                                                     int64_t n1, int64_t n2, int64_t n3,
                                                     int64_t s0, int64_t s1, int64_t s2,
                                                     int64_t s3, void* dst, int ddt, int64_t d0,
                                                     int64_t d1, int64_t d2, int64_t d3) {
  const int64_t n = n0 * n1 * n2 * n3;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t r = e;
    const int64_t i3 = r % n3;
    r /= n3;
    const int64_t i2 = r % n2;
    r /= n2;
    const int64_t i1 = r % n1, i0 = r / n1;
    const float v = load_f32(src, sdt, i0 * s0 + i1 * s1 + i2 * s2 + i3 * s3);
    const int64_t o = i0 * d0 + i1 * d1 + i2 * d2 + i3 * d3;
    if (ddt == kF16)
      static_cast<uint16_t*>(dst)[o] = f16_of(v);
    else if (ddt == kBF16)
      static_cast<uint16_t*>(dst)[o] = f32_to_bf16(v);
    else
      static_cast<float*>(dst)[o] = v;
  }
}

int grid_for(int64_t rows) {
  const int64_t t = (rows + kRows - 1) / kRows;
  return static_cast<int>(t < 2048 ? (t > 0 ? t : 1) : 2048);
}

}  // namespace

void launch_tq_encode(const TqEncodeArgs& a, hipStream_t st) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.H * a.Tc;
  if (rows <= 0) return;
  VKV_CHECK(a.D >= 2 && a.D <= 256, "TurboQuant head dims must be in [2, 256]");
  VKV_CHECK(a.bits >= 1 && a.bits <= 8, "TurboQuant index bits must be in [1, 8]");
  const size_t lds = static_cast<size_t>(kRows) * a.D * (4 + 1 + 1);
  const dim3 g(grid_for(rows)), b(kThreads);
  switch (a.D) {
    case 64: hipLaunchKernelGGL(tq_encode_kernel<64>, g, b, lds, st, a); break;
    case 128: hipLaunchKernelGGL(tq_encode_kernel<128>, g, b, lds, st, a); break;
    case 256: hipLaunchKernelGGL(tq_encode_kernel<256>, g, b, lds, st, a); break;
    default: hipLaunchKernelGGL(tq_encode_kernel<0>, g, b, lds, st, a); break;
  }
  VKV_HIP(hipGetLastError());
}

void launch_tq_decode(const TqDecodeArgs& a, hipStream_t st) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.H * a.Tc;
  if (rows <= 0) return;
  VKV_CHECK(a.D >= 2 && a.D <= 256, "TurboQuant head dims must be in [2, 256]");
  VKV_CHECK(a.bits >= 1 && a.bits <= 8, "TurboQuant index bits must be in [1, 8]");
  const size_t lds = static_cast<size_t>(kRows) * a.D * (4 + 1);
  const dim3 g(grid_for(rows)), b(kThreads);
  switch (a.D) {
    case 64: hipLaunchKernelGGL(tq_decode_kernel<64>, g, b, lds, st, a); break;
    case 128: hipLaunchKernelGGL(tq_decode_kernel<128>, g, b, lds, st, a); break;
    case 256: hipLaunchKernelGGL(tq_decode_kernel<256>, g, b, lds, st, a); break;
    default: hipLaunchKernelGGL(tq_decode_kernel<0>, g, b, lds, st, a); break;
  }
  VKV_HIP(hipGetLastError());
}

void launch_cast4d(const void* src, int sdt, const int64_t* shape, const int64_t* sstr, void* dst,
                   int ddt, const int64_t* dstr, hipStream_t st) {
  const int64_t n = shape[0] * shape[1] * shape[2] * shape[3];
  if (n <= 0) return;
  const int g = static_cast<int>(std::min<int64_t>((n + 255) / 256, 4096));
  hipLaunchKernelGGL(cast4d_kernel, dim3(g), dim3(256), 0, st, src, sdt, shape[0], shape[1],
                     shape[2], shape[3], sstr[0], sstr[1], sstr[2], sstr[3], dst, ddt, dstr[0],
                     dstr[1], dstr[2], dstr[3]);
  VKV_HIP(hipGetLastError());
}

}  // namespace vkv
