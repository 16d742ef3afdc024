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
#include <hip/hip_ext.h>

#include <algorithm>

#include "vkv_device.h"
#include "vkv_internal.h"

#pragma clang fp contract(off)

namespace vkv {
namespace {

constexpr int kRows = kTqTileRows;
constexpr int kThreads = 256;
static_assert(kRows * 8 == kThreads, "row sums use eight lanes per row");

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

// Sum over the 8 lanes of an aligned lane group (every lane gets it).
__device__ __forceinline__ double group8_sum_d(double v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  return v;
}

// The blockwise butterfly of TQHadamard.hadamardTransform over a tile of
// `rows` vectors held in LDS (row stride D): every block (n = 2^L values)
// runs its stages (a + b, a - b) on pairs (g 2h + j, g 2h + h + j), then
// scales by its f32 1 / sqrt(n).  Block sizes are powers of two, so every
// index below is a shift or a mask.
__device__ void hadamard_tile(float* y, int rows, int D, const TqBlocks& bl) {
  const int tid = threadIdx.x;
  for (int b = 0; b < bl.n; ++b) {
    const int n = bl.size[b], off = bl.off[b];
    const int L = __builtin_ctz(n);
    if (L == 0) continue;  // a block of one value: the transform is the identity
    for (int s = 0; s < L; ++s) {
      __syncthreads();
      const int h = 1 << s;
      for (int p = tid; p < (rows << (L - 1)); p += kThreads) {
        const int r = p >> (L - 1), q = p & ((1 << (L - 1)) - 1);
        float* v = y + r * D + off + ((q >> s) << (s + 1)) + (q & (h - 1));
        const float a = v[0], c = v[h];
        v[0] = a + c;
        v[h] = a - c;
      }
    }
    __syncthreads();
    const float sc = bl.scale[b];
    for (int p = tid; p < (rows << L); p += kThreads) {
      float* v = y + (p >> L) * D + off + (p & (n - 1));
      *v = *v * sc;
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
    // thread: 4 adjacent columns x RPT rows; a wave's lanes share rows in
    // groups, so the row operand is an LDS broadcast read
    constexpr int C = 4;
    constexpr int GC = DT / C;             // column groups
    constexpr int GR = kThreads / GC;      // row groups
    constexpr int RPT = kRows / GR;        // rows per thread
    const int j0 = (tid % GC) * C, rg = tid / GC;
    float acc[RPT][C];
#pragma unroll
    for (int k = 0; k < RPT; ++k)
#pragma unroll
      for (int c = 0; c < C; ++c) acc[k][c] = 0.0f;
#pragma unroll 2
    for (int i0 = 0; i0 < DT; i0 += 4) {
      float4 m[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) m[u] = *reinterpret_cast<const float4*>(M + (i0 + u) * DT + j0);
#pragma unroll
      for (int k = 0; k < RPT; ++k) {
        const int r = rg * RPT + k;
        float x[4];
        if constexpr (SGN) {
          const uint32_t w = *reinterpret_cast<const uint32_t*>(sa + r * DT + i0);
#pragma unroll
          for (int u = 0; u < 4; ++u) x[u] = ((w >> (8 * u)) & 0xffu) ? 1.0f : -1.0f;
        } else {
          const float4 v = *reinterpret_cast<const float4*>(a + r * DT + i0);
          x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
        }
        // each output's chain stays in i order
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          acc[k][0] = fmaf(x[u], m[u].x, acc[k][0]);
          acc[k][1] = fmaf(x[u], m[u].y, acc[k][1]);
          acc[k][2] = fmaf(x[u], m[u].z, acc[k][2]);
          acc[k][3] = fmaf(x[u], m[u].w, acc[k][3]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int r = rg * RPT + k;
      if (r < rows)
#pragma unroll
        for (int c = 0; c < C; ++c) f(r, j0 + c, acc[k][c]);
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

// The codec's tables in LDS: rotation signs, levels and boundaries.
struct TqLds {
  float signs[256];
  float cb[256];
  float bnd[256];
};

__device__ void load_tables(TqLds& t, const float* signs, const float* cb, const float* bnd,
                            int D, int nc) {
  for (int i = threadIdx.x; i < D; i += kThreads) t.signs[i] = signs[i];
  for (int i = threadIdx.x; i < nc; i += kThreads) t.cb[i] = cb[i];
  if (bnd)
    for (int i = threadIdx.x; i < nc - 1; i += kThreads) t.bnd[i] = bnd[i];
}

// Element offset of row r0 + r of a [B, H, Tc] row space inside a strided
// [B, H, T, D] array whose token axis starts at t0, for the tile's rows.
// The host keeps B * H * Tc below 2^31, so the row split is 32-bit.
__device__ void row_offsets(int64_t* off, int64_t r0, int nr, int H, int Tc, int t0, int64_t sb,
                            int64_t sh, int64_t st) {
  const int r = threadIdx.x;
  if (r < nr) {
    const uint32_t row = static_cast<uint32_t>(r0 + r);
    const uint32_t bh = row / static_cast<uint32_t>(Tc), t = row - bh * static_cast<uint32_t>(Tc);
    const uint32_t b = bh / static_cast<uint32_t>(H), h = bh - b * static_cast<uint32_t>(H);
    off[r] = static_cast<int64_t>(b) * sb + static_cast<int64_t>(h) * sh + (t0 + static_cast<int64_t>(t)) * st;
  }
}

template <int DT>
__global__ void __launch_bounds__(kThreads) tq_encode_kernel(TqEncodeArgs a) {
  extern __shared__ float lds[];
  const int D = DT > 0 ? DT : a.D;
  float* y = lds;                                                   // [kRows][D] f32
  uint8_t* codes = reinterpret_cast<uint8_t*>(y + kRows * D);       // [kRows][D]
  uint8_t* sg = codes + kRows * D;                                  // [kRows][D]
  __shared__ float den_s[kRows];
  __shared__ int64_t roff[kRows];
  __shared__ TqLds tb;
  const int tid = threadIdx.x;
  const int64_t rows = static_cast<int64_t>(a.B) * a.H * a.Tc, total = rows * D;
  const bool keys = a.St != nullptr;
  const int nb = a.nc - 1;
  load_tables(tb, a.signs, a.codebook, a.bounds, D, a.nc);
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRows; r0 < rows;
       r0 += static_cast<int64_t>(gridDim.x) * kRows) {
    const int nr = static_cast<int>(rows - r0 < kRows ? rows - r0 : kRows);
    row_offsets(roff, r0, nr, a.H, a.Tc, a.t0, a.sb, a.sh, a.st);
    __syncthreads();
    // 1. load the tile (rows past the end are zeros)
    for (int e = tid; e < kRows * D; e += kThreads) {
      const int r = e / D, i = e - r * D;
      y[e] = r < nr ? load_f32(a.x, a.dtype, roff[r] + i) : 0.0f;
    }
    __syncthreads();
    // 2. norm in T: T(sqrt(T(sum T(x_i^2)))), the divisor T(norm + T(1e-8));
    //    eight lanes per row, double sums
    {
      const int r = tid >> 3, part = tid & 7;
      double s = 0.0;
      for (int i = part; i < D; i += 8) {
        const float v = y[r * D + i];
        s += static_cast<double>(round_dt(v * v, a.dtype));
      }
      s = group8_sum_d(s);
      const float nrm = round_dt(sqrtf(round_dt(static_cast<float>(s), a.dtype)), a.dtype);
      if (part == 0) {
        den_s[r] = round_dt(nrm + round_dt(1e-8f, a.dtype), a.dtype);
        if (r < nr) a.vec_norms[r0 + r] = f16_of(nrm);
      }
    }
    __syncthreads();
    // 3. unit vector in T, times the rotation signs (f32), rotated
    for (int e = tid; e < kRows * D; e += kThreads) {
      const int r = e / D, i = e - r * D;
      y[e] = round_dt(y[e] / den_s[r], a.dtype) * tb.signs[i];
    }
    hadamard_tile(y, kRows, D, a.blocks);
    // 4. codes (boundaries exceeded); keys keep the residual y - level
    for (int e = tid; e < kRows * D; e += kThreads) {
      const float v = y[e];
      int idx = 0;
      for (int k = 0; k < nb; ++k) idx += v > tb.bnd[k];
      codes[e] = static_cast<uint8_t>(idx);
      if (keys) y[e] = v - tb.cb[idx];
    }
    __syncthreads();
    if (keys) {
      // 5. residual norm: f32(sum f32(r_i^2)) -> sqrt -> f16
      {
        const int r = tid >> 3, part = tid & 7;
        double s = 0.0;
        for (int i = part; i < D; i += 8) {
          const float v = y[r * D + i];
          s += static_cast<double>(v * v);
        }
        s = group8_sum_d(s);
        if (part == 0 && r < nr) a.res_norms[r0 + r] = f16_of(sqrtf(static_cast<float>(s)));
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

// The tile's elements [e0, e1) of a flat word array of `bits` values, into
// bytes: one thread per word.
__device__ void unpack_tile(const uint32_t* words, int64_t e0, int64_t e1, int bits,
                            uint8_t* out) {
  const int vpw = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  const int64_t w0 = e0 / vpw, w1 = (e1 - 1) / vpw;
  for (int64_t w = w0 + threadIdx.x; w <= w1; w += kThreads) {
    const uint32_t word = words[w];
    const int64_t base = w * vpw - e0;
    for (int k = 0; k < vpw; ++k) {
      const int64_t t = base + k;
      if (t >= 0 && t < e1 - e0) out[t] = static_cast<uint8_t>((word >> (k * bits)) & mask);
    }
  }
}

template <int DT>
__global__ void __launch_bounds__(kThreads) tq_decode_kernel(TqDecodeArgs a) {
  extern __shared__ float lds[];
  const int D = DT > 0 ? DT : a.D;
  float* z = lds;                                                   // [kRows][D]
  uint8_t* codes = reinterpret_cast<uint8_t*>(z + kRows * D);       // [kRows][D]
  uint8_t* sg = codes + kRows * D;                                  // [kRows][D]
  __shared__ int64_t roff[kRows];
  __shared__ float cr[kRows];
  __shared__ float vn[kRows];
  __shared__ TqLds tb;
  const int tid = threadIdx.x;
  const int64_t rows = static_cast<int64_t>(a.B) * a.H * a.Tc;
  const bool keys = a.S != nullptr;
  load_tables(tb, a.signs, a.codebook, nullptr, D, 1 << a.bits);
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRows; r0 < rows;
       r0 += static_cast<int64_t>(gridDim.x) * kRows) {
    const int nr = static_cast<int>(rows - r0 < kRows ? rows - r0 : kRows);
    row_offsets(roff, r0, nr, a.H, a.Tc, a.t0, a.osb, a.osh, a.ost);
    if (tid < nr) {
      vn[tid] = f16_to_f32(a.vec_norms[r0 + tid]);
      if (keys) cr[tid] = a.qs * f16_to_f32(a.res_norms[r0 + tid]);
    }
    const int64_t e0 = r0 * D, e1 = (r0 + nr) * D;
    unpack_tile(a.indices, e0, e1, a.bits, codes);
    if (keys) unpack_tile(a.qjl, e0, e1, 1, sg);
    __syncthreads();
    for (int e = tid; e < kRows * D; e += kThreads) z[e] = e < nr * D ? tb.cb[codes[e]] : 0.0f;
    if (keys) {
      for (int e = nr * D + tid; e < kRows * D; e += kThreads) sg[e] = 0;
      __syncthreads();
      // z += (sqrt(pi/2) / d * |r|) * (signs . S)
      tile_matmul<DT, true>(nullptr, sg, nr, D, a.S, [&](int r, int j, float v) {
        z[r * D + j] = z[r * D + j] + cr[r] * v;
      });
    }
    hadamard_tile(z, kRows, D, a.blocks);
    for (int e = tid; e < nr * D; e += kThreads) {
      const int r = e / D, i = e - r * D;
      const float w = z[e] * tb.signs[i] * vn[r];
      const uint16_t hv = f16_of(w);
      const int64_t o = roff[r] + i;
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
  VKV_CHECK(rows < (int64_t{1} << 31), "TurboQuant encodes fewer than 2^31 vectors per call");
  VKV_CHECK(a.D >= 2 && a.D <= 256, "TurboQuant head dims must be in [2, 256]");
  VKV_CHECK(a.bits >= 1 && a.bits <= 8, "TurboQuant index bits must be in [1, 8]");
  const size_t lds = static_cast<size_t>(kRows) * a.D * (4 + 1 + 1);
  const dim3 g(grid_for(rows)), b(kThreads);
  // the key launch (the QJL projection) is the one the timing aid records
  const TimedLaunch tl = a.St ? timing_prepare(kTimeTqEncode) : TimedLaunch{};
  switch (a.D) {
    case 64: hipExtLaunchKernelGGL(tq_encode_kernel<64>, g, b, lds, st, tl.start, tl.stop, 0, a); break;
    case 128: hipExtLaunchKernelGGL(tq_encode_kernel<128>, g, b, lds, st, tl.start, tl.stop, 0, a); break;
    case 256: hipExtLaunchKernelGGL(tq_encode_kernel<256>, g, b, lds, st, tl.start, tl.stop, 0, a); break;
    default: hipExtLaunchKernelGGL(tq_encode_kernel<0>, g, b, lds, st, tl.start, tl.stop, 0, a); break;
  }
  VKV_HIP(hipGetLastError());
  if (a.St) timing_commit(tl);
}

void launch_tq_decode(const TqDecodeArgs& a, hipStream_t st) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.H * a.Tc;
  if (rows <= 0) return;
  VKV_CHECK(rows < (int64_t{1} << 31), "TurboQuant decodes fewer than 2^31 vectors per call");
  VKV_CHECK(a.D >= 2 && a.D <= 256, "TurboQuant head dims must be in [2, 256]");
  VKV_CHECK(a.bits >= 1 && a.bits <= 8, "TurboQuant index bits must be in [1, 8]");
  const size_t lds = static_cast<size_t>(kRows) * a.D * (4 + 1 + 1);
  const dim3 g(grid_for(rows)), b(kThreads);
  const TimedLaunch tl = a.S ? timing_prepare(kTimeTqDecode) : TimedLaunch{};
  switch (a.D) {
    case 64: hipExtLaunchKernelGGL(tq_decode_kernel<64>, g, b, lds, st, tl.start, tl.stop, 0, a); break;
    case 128: hipExtLaunchKernelGGL(tq_decode_kernel<128>, g, b, lds, st, tl.start, tl.stop, 0, a); break;
    case 256: hipExtLaunchKernelGGL(tq_decode_kernel<256>, g, b, lds, st, tl.start, tl.stop, 0, a); break;
    default: hipExtLaunchKernelGGL(tq_decode_kernel<0>, g, b, lds, st, tl.start, tl.stop, 0, a); break;
  }
  VKV_HIP(hipGetLastError());
  if (a.S) timing_commit(tl);
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
