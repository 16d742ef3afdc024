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
// A workgroup of 256 threads takes tiles of 32 vectors.  Head dims 64, 128
// and 256 (one Hadamard block) take the row kernels, which keep each vector
// in the registers of eight lanes (tq_encode_rows / tq_decode_rows); other
// dims take the tile kernels, which stage the tile in LDS.  The two matrix
// products run as f32 fused multiply-add chains in index order (register
// tiles of outputs, the matrix read from L2), the row sums in double; the
// same orders are what the CPU restatement fixes, so the codes, signs,
// norms and decoded values are bit-exact with it.  Contraction is off in
// this file: every other product and sum rounds as the reference writes it.
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

// ---------------------------------------------------------------------------
// Row kernels for head dims 64, 128 and 256 (one Hadamard block of D
// values).  Eight adjacent lanes hold a vector, lane p the E = D / 8
// contiguous values [p E, p E + E) in registers: the butterflies with h < E
// run inside a lane, those with h = E, 2E, 4E between lanes p and p ^ h / E
// (DPP moves), so the rotation needs no LDS and no barrier.  Every value is
// formed by the same operation on the same operands as in the tile kernels
// above (the norms' double sums take their terms in another order; a sum of
// at most 256 f32 terms is exact in double unless they span more than 29
// binades, so its f32 rounding is the same).  LDS keeps only the bytes to
// pack or unpack and, for keys, the projection's operand rows.

// The value of lane (lane ^ M) for M in {1, 2, 4}: the partner inside an
// aligned group of eight lanes.
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  const int i = __float_as_int(v);
  if constexpr (M == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(i, 0xB1, 0xF, 0xF, true));
  if constexpr (M == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(i, 0x4E, 0xF, 0xF, true));
  // lane ^ 4 = (lane ^ 3) ^ 7: a quad reversal, then the half-row mirror
  const int t = __builtin_amdgcn_mov_dpp(i, 0x1B, 0xF, 0xF, true);
  return __int_as_float(__builtin_amdgcn_mov_dpp(t, 0x141, 0xF, 0xF, true));
}

// One butterfly stage between lanes p and p ^ M: the lower lane keeps
// a + c, the upper a - c (a the lower lane's value, c the upper's).  The
// product by +-1 is exact, so the fma rounds the same sum or difference.
template <int M, int E>
__device__ __forceinline__ void cross_stage(float (&x)[E], int part) {
  const float s = (part & M) ? -1.0f : 1.0f;
#pragma unroll
  for (int k = 0; k < E; ++k) x[k] = fmaf(x[k], s, lane_xor<M>(x[k]));
}

// hadamardTransform of one block of D = 8 E values held as above: stages
// h = 1, 2, ..., D / 2 in order, then times the block's f32 1 / sqrt(D).
template <int E>
__device__ __forceinline__ void row_butterflies(float (&x)[E], int part, float scale) {
#pragma unroll
  for (int h = 1; h < E; h <<= 1)
#pragma unroll
    for (int k = 0; k < E; ++k)
      if (!(k & h)) {
        const float a = x[k], c = x[k + h];
        x[k] = a + c;
        x[k + h] = a - c;
      }
  cross_stage<1>(x, part);
  cross_stage<2>(x, part);
  cross_stage<4>(x, part);
#pragma unroll
  for (int k = 0; k < E; ++k) x[k] = x[k] * scale;
}

// Element offset of row `row` of a [B, H, Tc] row space inside a strided
// [B, H, T, D] array whose token axis starts at t0 (row < 2^31).
__device__ __forceinline__ int64_t row_offset(int64_t row, int H, int Tc, int t0, int64_t sb,
                                              int64_t sh, int64_t st) {
  const uint32_t rw = static_cast<uint32_t>(row);
  const uint32_t bh = rw / static_cast<uint32_t>(Tc), t = rw - bh * static_cast<uint32_t>(Tc);
  const uint32_t b = bh / static_cast<uint32_t>(H), h = bh - b * static_cast<uint32_t>(H);
  return static_cast<int64_t>(b) * sb + static_cast<int64_t>(h) * sh +
         (t0 + static_cast<int64_t>(t)) * st;
}

// E contiguous values of dtype dt from element offset `off` (16-byte
// aligned: the launcher checks the base and the strides) as f32.
template <int E>
__device__ __forceinline__ void load_run(const void* p, int dt, int64_t off, float (&x)[E]) {
  if (dt == kF32) {
    const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + off);
#pragma unroll
    for (int u = 0; u < E / 4; ++u) {
      const float4 v = q[u];
      x[4 * u] = v.x; x[4 * u + 1] = v.y; x[4 * u + 2] = v.z; x[4 * u + 3] = v.w;
    }
  } else {
    const uint4* q = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + off);
    const bool bf = dt == kBF16;
#pragma unroll
    for (int u = 0; u < E / 8; ++u) {
      const uint4 v = q[u];
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint16_t lo = static_cast<uint16_t>(w[c]), hi = static_cast<uint16_t>(w[c] >> 16);
        x[8 * u + 2 * c] = bf ? bf16_to_f32(lo) : f16_to_f32(lo);
        x[8 * u + 2 * c + 1] = bf ? bf16_to_f32(hi) : f16_to_f32(hi);
      }
    }
  }
}

// The flat word range of a tile: rows [r0, r0 + nr) of D values hold
// elements [r0 D, (r0 + nr) D), words from w0 on, the first element `lead`
// values into its word (32-bit arithmetic: r0 < 2^31, D <= 256).
struct TileWords {
  int64_t w0;
  int lead, n, nw;
};
__device__ __forceinline__ TileWords tile_words(int64_t r0, int nr, int D, int vpw) {
  const uint32_t q = static_cast<uint32_t>(r0) / static_cast<uint32_t>(vpw);
  const uint32_t rem = static_cast<uint32_t>(r0) - q * static_cast<uint32_t>(vpw);
  TileWords t;
  t.w0 = static_cast<int64_t>(q) * D + static_cast<int64_t>(rem * D / vpw);
  t.lead = static_cast<int>(rem * D % vpw);
  t.n = nr * D;
  t.nw = (t.lead + t.n + vpw - 1) / vpw;
  return t;
}

// pack_tile for the row kernels: words that start and end inside the tile
// (or end the tensor) are stored, the rest OR-ed into the zeroed output.
// With a power-of-two width no word crosses a row, so the bytes are read
// four at a time.
__device__ void pack_rows(const uint8_t* vals, int64_t r0, int nr, int D, bool last, int bits,
                          uint32_t* out) {
  const int vpw = 32 / bits;
  const TileWords tw = tile_words(r0, nr, D, vpw);
  if ((vpw & 3) == 0 && tw.lead == 0 && D % vpw == 0) {
    for (int lw = threadIdx.x; lw < tw.nw; lw += kThreads) {
      const uint32_t* v4 = reinterpret_cast<const uint32_t*>(vals + lw * vpw);
      uint32_t word = 0;
      for (int k = 0; k < vpw / 4; ++k) {
        const uint32_t v = v4[k];
        const uint32_t c = (v & 0xffu) | (((v >> 8) & 0xffu) << bits) |
                           (((v >> 16) & 0xffu) << (2 * bits)) | ((v >> 24) << (3 * bits));
        word |= c << (4 * k * bits);
      }
      out[tw.w0 + lw] = word;
    }
    return;
  }
  for (int lw = threadIdx.x; lw < tw.nw; lw += kThreads) {
    const int base = lw * vpw - tw.lead;
    uint32_t word = 0;
    for (int k = 0; k < vpw; ++k) {
      const int t = base + k;
      if (t >= 0 && t < tw.n) word |= static_cast<uint32_t>(vals[t]) << (k * bits);
    }
    if (base >= 0 && (base + vpw <= tw.n || last))
      out[tw.w0 + lw] = word;
    else if (word)
      atomicOr(out + tw.w0 + lw, word);
  }
}

// unpack_tile for the row kernels (bytes of the tile's elements).
__device__ void unpack_rows(const uint32_t* words, int64_t r0, int nr, int D, int bits,
                            uint8_t* out) {
  const int vpw = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  const TileWords tw = tile_words(r0, nr, D, vpw);
  if ((vpw & 3) == 0 && tw.lead == 0 && D % vpw == 0) {
    for (int lw = threadIdx.x; lw < tw.nw; lw += kThreads) {
      const uint32_t word = words[tw.w0 + lw];
      uint32_t* o4 = reinterpret_cast<uint32_t*>(out + lw * vpw);
      for (int k = 0; k < vpw / 4; ++k) {
        const uint32_t v = word >> (4 * k * bits);
        o4[k] = (v & mask) | (((v >> bits) & mask) << 8) | (((v >> (2 * bits)) & mask) << 16) |
                (((v >> (3 * bits)) & mask) << 24);
      }
    }
    return;
  }
  for (int lw = threadIdx.x; lw < tw.nw; lw += kThreads) {
    const uint32_t word = words[tw.w0 + lw];
    const int base = lw * vpw - tw.lead;
    for (int k = 0; k < vpw; ++k) {
      const int t = base + k;
      if (t >= 0 && t < tw.n) out[t] = static_cast<uint8_t>((word >> (k * bits)) & mask);
    }
  }
}

// The tile's QJL sign bits as +-1.0f (the projection's left operand): one
// thread per word, D a multiple of 32 so words never cross a tile.
__device__ void unpack_signs_rows(const uint32_t* words, int64_t r0, int nr, int D, float* out) {
  const int64_t w0 = r0 * (D / 32);
  const int nw = nr * (D / 32);
  for (int lw = threadIdx.x; lw < nw; lw += kThreads) {
    const uint32_t word = words[w0 + lw];
    float4* o4 = reinterpret_cast<float4*>(out + lw * 32);
#pragma unroll
    for (int k = 0; k < 8; ++k)
      o4[k] = make_float4((word >> (4 * k)) & 1u ? 1.0f : -1.0f,
                          (word >> (4 * k + 1)) & 1u ? 1.0f : -1.0f,
                          (word >> (4 * k + 2)) & 1u ? 1.0f : -1.0f,
                          (word >> (4 * k + 3)) & 1u ? 1.0f : -1.0f);
  }
}

template <int D, bool KEYS>
__global__ void __launch_bounds__(kThreads) tq_encode_rows(TqEncodeArgs a) {
  constexpr int E = D / 8;
  extern __shared__ float lds[];
  uint8_t* codes = reinterpret_cast<uint8_t*>(lds);          // [kRows][D]
  uint8_t* sg = codes + kRows * D;                            // keys: [kRows][D]
  float* y = reinterpret_cast<float*>(sg + kRows * D);        // keys: [kRows][D] residuals
  __shared__ float cb_s[256], bnd_s[256];
  const int tid = threadIdx.x, r = tid >> 3, part = tid & 7;
  const int64_t rows = static_cast<int64_t>(a.B) * a.H * a.Tc;
  constexpr bool keys = KEYS;
  const int nb = a.nc - 1;
  for (int i = tid; i < a.nc; i += kThreads) cb_s[i] = a.codebook[i];
  for (int i = tid; i < nb; i += kThreads) bnd_s[i] = a.bounds[i];
  float rs[E];
#pragma unroll
  for (int k = 0; k < E; ++k) rs[k] = a.signs[part * E + k];
  const float scale = a.blocks.scale[0];
  const float eps = round_dt(1e-8f, a.dtype);
  __syncthreads();
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRows; r0 < rows;
       r0 += static_cast<int64_t>(gridDim.x) * kRows) {
    const int nr = static_cast<int>(rows - r0 < kRows ? rows - r0 : kRows);
    const bool live = r < nr;
    // 1. the lane's run of the vector (rows past the end are zeros)
    float x[E];
    if (live) {
      load_run<E>(a.x, a.dtype,
                  row_offset(r0 + r, a.H, a.Tc, a.t0, a.sb, a.sh, a.st) + part * E, x);
    } else {
#pragma unroll
      for (int k = 0; k < E; ++k) x[k] = 0.0f;
    }
    // 2. norm in T, the divisor T(norm + T(1e-8))
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < E; ++k) s += static_cast<double>(round_dt(x[k] * x[k], a.dtype));
    s = group8_sum_d(s);
    const float nrm = round_dt(sqrtf(round_dt(static_cast<float>(s), a.dtype)), a.dtype);
    const float den = round_dt(nrm + eps, a.dtype);
    if (part == 0 && live) a.vec_norms[r0 + r] = f16_of(nrm);
    // 3. unit vector in T, times the rotation signs, rotated
#pragma unroll
    for (int k = 0; k < E; ++k) x[k] = round_dt(x[k] / den, a.dtype) * rs[k];
    row_butterflies<E>(x, part, scale);
    // 4. codes; keys keep the residual y - level
    int idx[E];
#pragma unroll
    for (int k = 0; k < E; ++k) idx[k] = 0;
    for (int b = 0; b < nb; ++b) {
      const float bv = bnd_s[b];
#pragma unroll
      for (int k = 0; k < E; ++k) idx[k] += x[k] > bv;
    }
    {
      uint32_t* c4 = reinterpret_cast<uint32_t*>(codes + r * D + part * E);
#pragma unroll
      for (int u = 0; u < E / 4; ++u)
        c4[u] = static_cast<uint32_t>(idx[4 * u]) | (static_cast<uint32_t>(idx[4 * u + 1]) << 8) |
                (static_cast<uint32_t>(idx[4 * u + 2]) << 16) |
                (static_cast<uint32_t>(idx[4 * u + 3]) << 24);
    }
    if constexpr (keys) {
      // 5. residual norm: f32(sum f32(r_i^2)) -> sqrt -> f16
      double q = 0.0;
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const float v = x[k] - cb_s[idx[k]];
        x[k] = v;
        q += static_cast<double>(v * v);
      }
      q = group8_sum_d(q);
      if (part == 0 && live) a.res_norms[r0 + r] = f16_of(sqrtf(static_cast<float>(q)));
      float4* y4 = reinterpret_cast<float4*>(y + r * D + part * E);
#pragma unroll
      for (int u = 0; u < E / 4; ++u)
        y4[u] = make_float4(x[4 * u], x[4 * u + 1], x[4 * u + 2], x[4 * u + 3]);
    }
    __syncthreads();
    // 6. projection through S (S^T as the right operand), signs p >= 0
    if constexpr (keys)
      tile_matmul<D, false>(y, nullptr, nr, D, a.St,
                            [&](int rr, int j, float v) { sg[rr * D + j] = v >= 0.0f; });
    // 7. pack codes and signs into the flat words
    const bool last = r0 + nr == rows;
    pack_rows(codes, r0, nr, D, last, a.bits, a.indices);
    if constexpr (keys) pack_rows(sg, r0, nr, D, last, 1, a.qjl);
    __syncthreads();
  }
}

template <int D, bool KEYS>
__global__ void __launch_bounds__(kThreads) tq_decode_rows(TqDecodeArgs a) {
  constexpr int E = D / 8;
  extern __shared__ float lds[];
  uint8_t* codes = reinterpret_cast<uint8_t*>(lds);          // [kRows][D]
  float* sgf = reinterpret_cast<float*>(codes + kRows * D);   // keys: [kRows][D] +-1
  float* z = sgf + kRows * D;                                 // keys: [kRows][D]
  __shared__ float cb_s[256], cr_s[kRows];
  const int tid = threadIdx.x, r = tid >> 3, part = tid & 7;
  const int64_t rows = static_cast<int64_t>(a.B) * a.H * a.Tc;
  constexpr bool keys = KEYS;
  for (int i = tid; i < (1 << a.bits); i += kThreads) cb_s[i] = a.codebook[i];
  float rs[E];
#pragma unroll
  for (int k = 0; k < E; ++k) rs[k] = a.signs[part * E + k];
  const float scale = a.blocks.scale[0];
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRows; r0 < rows;
       r0 += static_cast<int64_t>(gridDim.x) * kRows) {
    const int nr = static_cast<int>(rows - r0 < kRows ? rows - r0 : kRows);
    const bool live = r < nr;
    unpack_rows(a.indices, r0, nr, D, a.bits, codes);
    if constexpr (keys) {
      unpack_signs_rows(a.qjl, r0, nr, D, sgf);
      if (tid < nr) cr_s[tid] = a.qs * f16_to_f32(a.res_norms[r0 + tid]);
    }
    const float vn = live ? f16_to_f32(a.vec_norms[r0 + r]) : 0.0f;
    __syncthreads();
    float x[E];
    if constexpr (keys) {
      // z = level + (sqrt(pi/2) / d * |r|) * (signs . S); fma(+-1, S, q) is
      // the sum or difference the reference's sign product rounds.  The rows
      // past the end read stale operands and are not kept.
      tile_matmul<D, false>(sgf, nullptr, nr, D, a.S, [&](int rr, int j, float v) {
        z[rr * D + j] = cb_s[codes[rr * D + j]] + cr_s[rr] * v;
      });
      const float4* z4 = reinterpret_cast<const float4*>(z + r * D + part * E);
#pragma unroll
      for (int u = 0; u < E / 4; ++u) {
        const float4 v = live ? z4[u] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        x[4 * u] = v.x; x[4 * u + 1] = v.y; x[4 * u + 2] = v.z; x[4 * u + 3] = v.w;
      }
    } else {
      const uint32_t* c4 = reinterpret_cast<const uint32_t*>(codes + r * D + part * E);
#pragma unroll
      for (int u = 0; u < E / 4; ++u) {
        const uint32_t w = live ? c4[u] : 0u;
#pragma unroll
        for (int c = 0; c < 4; ++c) x[4 * u + c] = live ? cb_s[(w >> (8 * c)) & 0xffu] : 0.0f;
      }
    }
    row_butterflies<E>(x, part, scale);
    if (live) {
      const int64_t o = row_offset(r0 + r, a.H, a.Tc, a.t0, a.osb, a.osh, a.ost) + part * E;
      uint16_t hv[E];
#pragma unroll
      for (int k = 0; k < E; ++k) hv[k] = f16_of(x[k] * rs[k] * vn);
      if (a.out_dtype == kF16) {
        uint4* q = reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.out) + o);
#pragma unroll
        for (int u = 0; u < E / 8; ++u) {
          uint32_t w[4];
#pragma unroll
          for (int c = 0; c < 4; ++c)
            w[c] = static_cast<uint32_t>(hv[8 * u + 2 * c]) |
                   (static_cast<uint32_t>(hv[8 * u + 2 * c + 1]) << 16);
          q[u] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      } else {
        float4* q = reinterpret_cast<float4*>(static_cast<float*>(a.out) + o);
#pragma unroll
        for (int u = 0; u < E / 4; ++u)
          q[u] = make_float4(f16_to_f32(hv[4 * u]), f16_to_f32(hv[4 * u + 1]),
                             f16_to_f32(hv[4 * u + 2]), f16_to_f32(hv[4 * u + 3]));
      }
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

// Zeros over `rows` runs of `run` units of T, `pitch` units apart.
template <class T>
__global__ void __launch_bounds__(256) zero_runs_kernel(T* base, int64_t pitch, int64_t run,
                                                        int64_t rows) {
  const int64_t n = run * rows;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = e / run;
    base[r * pitch + (e - r * run)] = T{};
  }
}

int grid_for(int64_t rows) {
  const int64_t t = (rows + kRows - 1) / kRows;
  return static_cast<int>(t < 2048 ? (t > 0 ? t : 1) : 2048);
}

// The row kernels take head dims 64, 128 and 256 (one Hadamard block) over
// an array whose base and strides keep every lane's run 16-byte aligned.
bool rows_kernel_fits(int D, const TqBlocks& bl, const void* base, int es, int64_t s0, int64_t s1,
                      int64_t s2) {
  if (!(D == 64 || D == 128 || D == 256) || bl.n != 1) return false;
  return reinterpret_cast<uintptr_t>(base) % 16 == 0 && (s0 * es) % 16 == 0 &&
         (s1 * es) % 16 == 0 && (s2 * es) % 16 == 0;
}

}  // namespace

void launch_tq_encode(const TqEncodeArgs& a, hipStream_t st) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.H * a.Tc;
  if (rows <= 0) return;
  VKV_CHECK(rows < (int64_t{1} << 31), "TurboQuant encodes fewer than 2^31 vectors per call");
  VKV_CHECK(a.D >= 2 && a.D <= 256, "TurboQuant head dims must be in [2, 256]");
  VKV_CHECK(a.bits >= 1 && a.bits <= 8, "TurboQuant index bits must be in [1, 8]");
  const dim3 g(grid_for(rows)), b(kThreads);
  // the key launch (the QJL projection) is the one the timing aid records
  const TimedLaunch tl = a.St ? timing_prepare(kTimeTqEncode) : TimedLaunch{};
  const int es = a.dtype == kF32 ? 4 : 2;
  if (rows_kernel_fits(a.D, a.blocks, a.x, es, a.sb, a.sh, a.st)) {
    const size_t lds = static_cast<size_t>(kRows) * a.D * (a.St ? 6 : 1);
    switch (a.D) {
      case 64: a.St ? hipExtLaunchKernelGGL((tq_encode_rows<64, true>), g, b, lds, st, tl.start, tl.stop, 0, a)
              : hipExtLaunchKernelGGL((tq_encode_rows<64, false>), g, b, lds, st, tl.start, tl.stop, 0, a);
      break;
      case 128: a.St ? hipExtLaunchKernelGGL((tq_encode_rows<128, true>), g, b, lds, st, tl.start, tl.stop, 0, a)
              : hipExtLaunchKernelGGL((tq_encode_rows<128, false>), g, b, lds, st, tl.start, tl.stop, 0, a);
      break;
      default: a.St ? hipExtLaunchKernelGGL((tq_encode_rows<256, true>), g, b, lds, st, tl.start, tl.stop, 0, a)
              : hipExtLaunchKernelGGL((tq_encode_rows<256, false>), g, b, lds, st, tl.start, tl.stop, 0, a);
      break;
    }
  } else {
    const size_t lds = static_cast<size_t>(kRows) * a.D * (4 + 1 + 1);
    hipExtLaunchKernelGGL(tq_encode_kernel<0>, g, b, lds, st, tl.start, tl.stop, 0, a);
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
  const dim3 g(grid_for(rows)), b(kThreads);
  const TimedLaunch tl = a.S ? timing_prepare(kTimeTqDecode) : TimedLaunch{};
  const int es = a.out_dtype == kF32 ? 4 : 2;
  if (rows_kernel_fits(a.D, a.blocks, a.out, es, a.osb, a.osh, a.ost)) {
    const size_t lds = static_cast<size_t>(kRows) * a.D * (a.S ? 9 : 1);
    switch (a.D) {
      case 64: a.S ? hipExtLaunchKernelGGL((tq_decode_rows<64, true>), g, b, lds, st, tl.start, tl.stop, 0, a)
              : hipExtLaunchKernelGGL((tq_decode_rows<64, false>), g, b, lds, st, tl.start, tl.stop, 0, a);
      break;
      case 128: a.S ? hipExtLaunchKernelGGL((tq_decode_rows<128, true>), g, b, lds, st, tl.start, tl.stop, 0, a)
              : hipExtLaunchKernelGGL((tq_decode_rows<128, false>), g, b, lds, st, tl.start, tl.stop, 0, a);
      break;
      default: a.S ? hipExtLaunchKernelGGL((tq_decode_rows<256, true>), g, b, lds, st, tl.start, tl.stop, 0, a)
              : hipExtLaunchKernelGGL((tq_decode_rows<256, false>), g, b, lds, st, tl.start, tl.stop, 0, a);
      break;
    }
  } else {
    const size_t lds = static_cast<size_t>(kRows) * a.D * (4 + 1 + 1);
    hipExtLaunchKernelGGL(tq_decode_kernel<0>, g, b, lds, st, tl.start, tl.stop, 0, a);
  }
  VKV_HIP(hipGetLastError());
  if (a.S) timing_commit(tl);
}

void launch_zero_runs(void* base, int64_t pitch_bytes, int64_t run_bytes, int64_t rows,
                      hipStream_t st) {
  if (run_bytes <= 0 || rows <= 0) return;
  VKV_CHECK(pitch_bytes % 2 == 0 && run_bytes % 2 == 0 && reinterpret_cast<uintptr_t>(base) % 2 == 0,
            "zeroed runs are whole 2-byte units");
  const bool wide = pitch_bytes % 16 == 0 && run_bytes % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(base) % 16 == 0;
  const int64_t unit = wide ? 16 : 2, n = run_bytes / unit * rows;
  const int g = static_cast<int>(std::min<int64_t>((n + 255) / 256, 4096));
  if (wide)
    hipLaunchKernelGGL(zero_runs_kernel<uint4>, dim3(g), dim3(256), 0, st, static_cast<uint4*>(base),
                       pitch_bytes / 16, run_bytes / 16, rows);
  else
    hipLaunchKernelGGL(zero_runs_kernel<uint16_t>, dim3(g), dim3(256), 0, st,
                       static_cast<uint16_t*>(base), pitch_bytes / 2, run_bytes / 2, rows);
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
