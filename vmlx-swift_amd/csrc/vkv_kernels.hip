// vkv_kernels.hip -- gfx950 kernels of the KV-cache engine: affine
// quantize-on-append (dense and paged, bit-exact with the reference
// quantizer), scatter/gather, dequant-on-read, strided copies, and the
// generic split-K decode attention used for float and quantized caches.
//
// Reference arithmetic: Source/Cmlx/mlx-generated/metal/quantized.h:2393-2560
// (affine quantize / dequantize) and sdpa_vector.h:15-394 (decode SDPA and
// its two-pass combine); Libraries/MLXLMCommon/KVCache.swift:1909-1997
// (quantized SDPA semantics).
#include "vkv_device.h"
#include "vkv_internal.h"
#include "vkv_kvread.h"
#include <hip/hip_ext.h>

#include <algorithm>

namespace vkv {

// ----------------------------------------------------------------- helpers

__device__ __forceinline__ const uint8_t* row_ptr(const RowSrc& s, int64_t row, int esize) {
  int64_t i2 = row % s.e2;
  int64_t r1 = row / s.e2;
  int64_t i1 = r1 % s.e1;
  int64_t i0 = r1 / s.e1;
  return static_cast<const uint8_t*>(s.ptr) + (i0 * s.s0 + i1 * s.s1 + i2 * s.s2) * esize;
}

// Slot (block * block_size + offset) of paged token n; < 0 means skip (so
// does an explicit slot past the pool, which would write outside it).
__device__ __forceinline__ int64_t token_slot(const RowDst& d, int64_t n) {
  if (d.slots) {
    const int64_t s = d.slots[n];
    return (d.slot_limit > 0 && s >= d.slot_limit) ? -1 : s;
  }
  int64_t b = n / d.seq_S;
  int64_t pos = d.start + n % d.seq_S;
  int32_t blk = d.table[b * d.table_stride + pos / d.block_size];
  if (blk < 0) return -1;
  return static_cast<int64_t>(blk) * d.block_size + pos % d.block_size;
}

template <int DT>
__device__ __forceinline__ void load8(const uint8_t* p, float* v) {
  using E = Elem<DT>;
  const typename E::T* q = reinterpret_cast<const typename E::T*>(p);
#pragma unroll
  for (int i = 0; i < 8; i++) v[i] = E::load(q + i);
}

// Store the 8 codes of dims [8j, 8j+8) of token `tib` into a paged chunk
// (format in vkv_device.h).  V codes of one word belong to 8 different
// tokens, so a 4-bit V store is a read-modify-write done with two atomics on
// the containing word (other tokens' nibbles may be written concurrently).
template <int BITS>
__device__ __forceinline__ void store_chunk_codes(uint8_t* chunk, const RowDst& dst, int tib, int j,
                                                  int D, const uint32_t* code) {
  uint8_t* c = chunk + dst.c_off;
  if (!dst.is_v) {
    if constexpr (BITS == 4) {
      uint32_t w = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) w |= code[i] << (4 * i);
      *reinterpret_cast<uint32_t*>(c + qk_word_off(tib, j, D, 4)) = w;
    } else {
      const uint32_t w0 = code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
      const uint32_t w1 = code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24);
      *reinterpret_cast<uint32_t*>(c + qk_word_off(tib, 2 * j, D, 8)) = w0;
      *reinterpret_cast<uint32_t*>(c + qk_word_off(tib, 2 * j + 1, D, 8)) = w1;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      int sh;
      const int64_t off = qv_word_off(tib, j * 8 + i, D, BITS, &sh);
      if constexpr (BITS == 8) {
        c[off + sh / 8] = static_cast<uint8_t>(code[i]);
      } else {
        uint32_t* word = reinterpret_cast<uint32_t*>(c + off);
        atomicAnd(word, ~(0xFu << sh));
        atomicOr(word, code[i] << sh);
      }
    }
  }
}

// ------------------------------------------------------- affine quantize
//
// One thread owns 8 consecutive values of a row; GROUP/8 neighbouring lanes
// form one quantization group and reduce min/max with xor-shuffles; the
// arithmetic is the reference's (affine_quantize8, quantized.h:2422-2458),
// scale/bias stored rounded to T (:2447-2450).
// mode 0 writes the reference layout; mode 1 writes a paged chunk (K rows
// token-major, V rows dim-major).
template <int DT, int BITS, int GROUP, int MODE>
__global__ void __launch_bounds__(256) quantize_rows_kernel(RowSrc src, RowDst dst, int64_t rows,
                                                            int D) {
  using E = Elem<DT>;
  constexpr int TEAM = GROUP / 8;
  const int tpr = D / 8;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = gtid / tpr;
  const int j = static_cast<int>(gtid % tpr);
  const bool active = row < rows;

  float v[8];
  if (active) {
    load8<DT>(row_ptr(src, row, E::kBytes) + static_cast<int64_t>(j) * 8 * E::kBytes, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = 0.0f;
  }
  uint32_t code[8];
  float scale, bias;
  affine_quantize8<DT, BITS, GROUP>(v, code, scale, bias);
  if (!active) return;
  const int G = D / GROUP;
  const int g = (j * 8) / GROUP;
  const bool group_leader = (j % TEAM) == 0;
  const typename E::T s_t = E::from_f32(scale);
  const typename E::T b_t = E::from_f32(bias);

  if constexpr (MODE == 0) {
    uint32_t* wq = static_cast<uint32_t*>(dst.wq) + row * (D * BITS / 32);
    if constexpr (BITS == 4) {
      uint32_t w = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) w |= code[i] << (4 * i);
      wq[j] = w;
    } else {
      uint32_t w0 = code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
      uint32_t w1 = code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24);
      wq[2 * j] = w0;
      wq[2 * j + 1] = w1;
    }
    if (group_leader) {
      static_cast<typename E::T*>(dst.scales)[row * G + g] = s_t;
      static_cast<typename E::T*>(dst.biases)[row * G + g] = b_t;
    }
  } else {
    const int64_t n = row / src.e2;
    const int64_t h = row % src.e2;
    const int64_t slot = token_slot(dst, n);
    if (slot < 0) return;
    const int64_t blk = slot / dst.block_size;
    const int tib = static_cast<int>(slot % dst.block_size);
    uint8_t* chunk = dst.base + blk * dst.block_bytes + h * dst.head_bytes;
    store_chunk_codes<BITS>(chunk, dst, tib, j, D, code);
    if (group_leader) {
      typename E::T* sbp = reinterpret_cast<typename E::T*>(chunk + dst.s_off);
      sbp[qsb_index(tib, dst.is_v, g, 0, dst.G, dst.keys_only)] = s_t;
      sbp[qsb_index(tib, dst.is_v, g, 1, dst.G, dst.keys_only)] = b_t;
    }
  }
}

// Paged append of K and V in one launch (Pool::append): block = 8
// consecutive tokens x HB heads x the D/8 threads of a row (256 threads);
// blockIdx.z selects K (0) or V (1).  The arithmetic is that of
// quantize_rows_kernel.  4-bit V words hold 8 tokens of one dim: when the
// block's 8 tokens fill exactly one aligned 8-token group of a block (a
// prefill chunk), the words are assembled in LDS and written with plain
// stores; otherwise (decode tokens of different sequences, ragged groups)
// each nibble is merged atomically.
template <int DT, int BITS, int GROUP>
__global__ void __launch_bounds__(256) append_affine_kernel(RowSrc sk, RowSrc sv, RowDst dk, RowDst dv,
                                                            int64_t ntok, int H, int D) {
  using E = Elem<DT>;
  constexpr int TEAM = GROUP / 8;
  const int which = blockIdx.z;
  const RowSrc src = which ? sv : sk;
  const RowDst dst = which ? dv : dk;
  const int tpr = D / 8, hb = 256 / (8 * tpr);
  const int tid = threadIdx.x;
  const int i = tid / (hb * tpr), hl = (tid / tpr) % hb, j = tid % tpr;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * 8 + i;
  const int h = blockIdx.y * hb + hl;
  const bool active = n < ntok && h < H;
  // the token's slot (a block-table read) goes out with the row's load
  const int64_t slot = active ? token_slot(dst, n) : -1;

  float v[8];
  if (active) {
    load8<DT>(row_ptr(src, n * H + h, E::kBytes) + static_cast<int64_t>(j) * 8 * E::kBytes, v);
  } else {
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = 0.0f;
  }
  uint32_t code[8];
  float scale, bias;
  affine_quantize8<DT, BITS, GROUP>(v, code, scale, bias);
  const int g = (j * 8) / GROUP;
  if (slot >= 0 && (j % TEAM) == 0) {
    uint8_t* chunk = dst.base + (slot / dst.block_size) * dst.block_bytes + h * dst.head_bytes;
    const int tib = static_cast<int>(slot % dst.block_size);
    typename E::T* sbp = reinterpret_cast<typename E::T*>(chunk + dst.s_off);
    sbp[qsb_index(tib, dst.is_v, g, 0, dst.G, dst.keys_only)] = E::from_f32(scale);
    sbp[qsb_index(tib, dst.is_v, g, 1, dst.G, dst.keys_only)] = E::from_f32(bias);
  }
  if (BITS == 8 || which == 0) {  // K words and 8-bit V bytes are whole stores
    if (slot >= 0) {
      uint8_t* chunk = dst.base + (slot / dst.block_size) * dst.block_bytes + h * dst.head_bytes;
      store_chunk_codes<BITS>(chunk, dst, static_cast<int>(slot % dst.block_size), j, D, code);
    }
    return;
  }
  // ---- 4-bit V
  __shared__ int64_t tok_slot[8];
  __shared__ uint8_t vcode[8][256];  // [token][head * D + dim], hb * D = 256
  if (hl == 0 && j == 0) tok_slot[i] = slot;  // hl 0: a head below H, so slot is n's
  __syncthreads();
  const int64_t s0 = tok_slot[0];
  bool aligned = s0 >= 0 && s0 % 8 == 0;
#pragma unroll
  for (int t = 1; t < 8; t++) aligned = aligned && tok_slot[t] == s0 + t;
  if (!aligned) {
    if (slot >= 0) {
      uint8_t* chunk = dst.base + (slot / dst.block_size) * dst.block_bytes + h * dst.head_bytes;
      store_chunk_codes<BITS>(chunk, dst, static_cast<int>(slot % dst.block_size), j, D, code);
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; e++) vcode[i][hl * D + 8 * j + e] = static_cast<uint8_t>(code[e]);
  __syncthreads();
  // thread (head hh, dim d) writes the word of the 8 tokens
  const int hh = tid / D, d = tid % D;
  if (tid < hb * D && blockIdx.y * hb + hh < H) {
    uint32_t w = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) w |= static_cast<uint32_t>(vcode[t][hh * D + d]) << (4 * t);
    uint8_t* chunk = dst.base + (s0 / dst.block_size) * dst.block_bytes +
                     static_cast<int64_t>(blockIdx.y * hb + hh) * dst.head_bytes;
    int sh;
    const int64_t off = qv_word_off(s0 % dst.block_size, d, D, 4, &sh);
    *reinterpret_cast<uint32_t*>(chunk + dst.c_off + off) = w;
  }
}

// Float rows: mode 0 copies to contiguous out (dst.wq), mode 1 scatters to
// paged chunks (token-major K or V at dst.c_off).
template <int ESIZE, int MODE>
__global__ void __launch_bounds__(256) copy_rows_kernel(RowSrc src, RowDst dst, int64_t rows, int D) {
  const int tpr = (D + 7) / 8;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = gtid / tpr;
  const int j = static_cast<int>(gtid % tpr);
  if (row >= rows) return;
  const uint8_t* s = row_ptr(src, row, ESIZE) + static_cast<int64_t>(j) * 8 * ESIZE;
  uint8_t* o;
  if constexpr (MODE == 0) {
    o = static_cast<uint8_t*>(dst.wq) + (row * D + j * 8) * ESIZE;
  } else {
    const int64_t n = row / src.e2;
    const int64_t h = row % src.e2;
    const int64_t slot = token_slot(dst, n);
    if (slot < 0) return;
    const int64_t blk = slot / dst.block_size;
    const int64_t tib = slot % dst.block_size;
    o = dst.base + blk * dst.block_bytes + h * dst.head_bytes + dst.c_off +
        (tib * D + j * 8) * ESIZE;
  }
  const int cnt = min(8, D - j * 8);
  if constexpr (ESIZE == 2) {
    const uint16_t* a = reinterpret_cast<const uint16_t*>(s);
    uint16_t* b = reinterpret_cast<uint16_t*>(o);
    for (int i = 0; i < cnt; i++) b[i] = a[i];
  } else {
    const uint32_t* a = reinterpret_cast<const uint32_t*>(s);
    uint32_t* b = reinterpret_cast<uint32_t*>(o);
    for (int i = 0; i < cnt; i++) b[i] = a[i];
  }
}

// quantized.h:2498-2560: out = scale * q + bias, here one fp32 fma rounded
// once to T.  Thread per 8 values, contiguous operands.
template <int DT, int BITS>
__global__ void __launch_bounds__(256) dequantize_kernel(const uint32_t* wq, const void* scales,
                                                         const void* biases, void* out, int64_t rows,
                                                         int D, int group) {
  using E = Elem<DT>;
  const int tpr = D / 8;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = gtid / tpr;
  const int j = static_cast<int>(gtid % tpr);
  if (row >= rows) return;
  const int G = D / group;
  const int g = j * 8 / group;
  const float s = E::load(static_cast<const typename E::T*>(scales) + row * G + g);
  const float b = E::load(static_cast<const typename E::T*>(biases) + row * G + g);
  const uint32_t* w = wq + row * (D * BITS / 32);
  typename E::T* o = static_cast<typename E::T*>(out) + row * D + j * 8;
  if constexpr (BITS == 4) {
    uint32_t x = w[j];
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = E::from_f32(fmaf(s, static_cast<float>((x >> (4 * i)) & 15u), b));
  } else {
    uint32_t x0 = w[2 * j], x1 = w[2 * j + 1];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      o[i] = E::from_f32(fmaf(s, static_cast<float>((x0 >> (8 * i)) & 255u), b));
      o[4 + i] = E::from_f32(fmaf(s, static_cast<float>((x1 >> (8 * i)) & 255u), b));
    }
  }
}

// --------------------------------------------------------------- gather
//
// Thread per (seq, head, token, 8 dims).  out_kind 0: values (dequantized
// when bits > 0) into [n,H,T,D] of dtype; out_kind 1: reference-layout codes.
template <int DT, int BITS, int KIND>
__global__ void __launch_bounds__(256) gather_kernel(GatherArgs g) {
  using E = Elem<DT>;
  const int tpr = (g.D + 7) / 8;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = gtid / tpr;  // (s, h, t)
  const int j = static_cast<int>(gtid % tpr);
  const int64_t total = static_cast<int64_t>(g.n_seqs) * g.H * g.T;
  if (row >= total) return;
  const int64_t t = row % g.T;
  const int64_t h = (row / g.T) % g.H;
  const int64_t s = row / (static_cast<int64_t>(g.T) * g.H);
  const int64_t len = g.kv.seq_lens ? g.kv.seq_lens[s] : g.kv.T;
  if (t + g.t_begin >= len) return;
  const TokLoc l = locate(g.kv, s, t + g.t_begin);
  const int d0 = j * 8;
  const int cnt = min(8, g.D - d0);
  if constexpr (KIND == 0) {
    typename E::T* o = static_cast<typename E::T*>(g.out) + row * g.D + d0;
    for (int i = 0; i < cnt; i++) o[i] = E::from_f32(kv_at<DT, BITS>(g.kv, l, h, d0 + i, g.which, g.group));
  } else {
    // codes of dims [d0, d0+8) re-packed little-endian into the reference layout
    uint32_t code[8];
    float s = 0.0f, b = 0.0f;
    for (int i = 0; i < 8; i++) code[i] = qcode<DT, BITS>(g.kv, l, h, d0 + i, g.which, g.group, &s, &b);
    // (the output row: token out_t0 + t of rows out_cap tokens long)
    const int64_t orow = (row / g.T) * (g.out_cap ? g.out_cap : g.T) + g.out_t0 + t;
    uint32_t* wq = static_cast<uint32_t*>(g.out) + orow * (g.D * BITS / 32);
    if constexpr (BITS == 4) {
      uint32_t w = 0;
      for (int i = 0; i < 8; i++) w |= code[i] << (4 * i);
      wq[j] = w;
    } else {
      wq[2 * j] = code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
      wq[2 * j + 1] = code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24);
    }
    if (d0 % g.group == 0) {
      // s and b of the group holding dims [d0, d0+8) (exact stored values)
      const int G = g.D / g.group;
      const int gi = d0 / g.group;
      static_cast<typename E::T*>(g.out_s)[orow * G + gi] = E::from_f32(s);
      static_cast<typename E::T*>(g.out_b)[orow * G + gi] = E::from_f32(b);
    }
  }
}

// Dequantizing gather, 8 dims per piece: one code word (4-bit) or two
// (8-bit) and one scale/bias pair (a group spans a multiple of 8 dims), then
// one 16-byte store of bf16/f16 (two of f32).  The values are those of
// gather_kernel<.., 0>: the fp32 scale * code + bias rounded to the dtype.
// blockIdx.y is the (seq, head) plane; with gridDim.z == 2, blockIdx.z picks
// K (into out) or V (into out_v) in one launch.  A thread takes
// kGatherPieces pieces 256 apart and issues all their loads before its first
// store (one piece measured fastest: more workgroups keep more loads in
// flight).  Needs D and group multiples of 8, 4-byte aligned code rows and a
// 16-byte aligned output (gather8_ok).
constexpr int kGatherPieces = 1;

template <int DT, int BITS>
__global__ void __launch_bounds__(256) gather_dequant8_kernel(GatherArgs g) {
  using E = Elem<DT>;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  const int tpr = g.D >> 3;
  const int plane = blockIdx.y, s = plane / g.H, h = plane - s * g.H;
  // tokens of this row in the window [t_begin, t_begin + T)
  const int len =
      min(g.T, static_cast<int>(g.kv.seq_lens ? g.kv.seq_lens[s] : g.kv.T) - g.t_begin);
  if (len <= 0) return;  // an empty sequence may own no block
  const KVSrc& kv = g.kv;
  const bool ko = kv.keys_only != 0;
  const int which = gridDim.z > 1 ? static_cast<int>(blockIdx.z) : g.which;
  void* const out = which && gridDim.z > 1 ? g.out_v : g.out;
  const int w = (which && !ko) ? 1 : 0;
  uint32_t w0[kGatherPieces], w1[kGatherPieces], c4[kGatherPieces][8];
  float sc[kGatherPieces], bi[kGatherPieces];
  bool live[kGatherPieces];
  int ti[kGatherPieces], d0[kGatherPieces];
#pragma unroll
  for (int k = 0; k < kGatherPieces; k++) {
    const int idx = (blockIdx.x * kGatherPieces + k) * 256 + static_cast<int>(threadIdx.x);
    ti[k] = idx / tpr;
    d0[k] = (idx - ti[k] * tpr) * 8;
    live[k] = ti[k] < len;
    // dead pieces load the window's first token (in bounds) and store nothing
    const int t = g.t_begin + (live[k] ? ti[k] : 0);
    TokLoc l;
    if (kv.table) {
      const int b = t / kv.block_size;
      l.blk = kv.table[static_cast<int64_t>(s) * kv.table_stride + b];
      l.tib = t - b * kv.block_size;
    } else {
      l.blk = s;
      l.tib = t;
    }
    const int gi = d0[k] / g.group;
    w0[k] = w1[k] = 0u;
    if (kv.qfmt) {
      const uint8_t* chunk = kv.base + l.blk * kv.block_bytes + h * kv.head_bytes;
      const typename E::T* sb = reinterpret_cast<const typename E::T*>(chunk + kv.sb_off);
      sc[k] = E::load(sb + qsb_index(l.tib, w, gi, 0, kv.G, ko));
      bi[k] = E::load(sb + qsb_index(l.tib, w, gi, 1, kv.G, ko));
      if (w == 0) {
        // the 8 dims are original word d0/8 (4-bit) or words d0/4, d0/4 + 1
        // (8-bit), which the chunk keeps side by side
        const uint32_t* p = reinterpret_cast<const uint32_t*>(
            chunk + kv.kc_off + qk_word_off(l.tib, d0[k] * BITS / 32, kv.D, BITS));
        w0[k] = p[0];
        if (BITS == 8) w1[k] = p[1];
      } else {
#pragma unroll
        for (int i = 0; i < 8; i++) {
          int sh;
          const uint32_t word = *reinterpret_cast<const uint32_t*>(
              chunk + kv.vc_off + qv_word_off(l.tib, d0[k] + i, kv.D, BITS, &sh));
          c4[k][i] = (word >> sh) & kMask;
        }
      }
    } else {
      const Comp& cc = which ? kv.vc : kv.kc;
      const Comp& scp = which ? kv.vs : kv.ks;
      const Comp& bcp = which ? kv.vb : kv.kb;
      sc[k] = E::load(reinterpret_cast<const typename E::T*>(at(scp, l, h)) + gi);
      bi[k] = E::load(reinterpret_cast<const typename E::T*>(at(bcp, l, h)) + gi);
      const uint32_t* p = reinterpret_cast<const uint32_t*>(at(cc, l, h) + d0[k] * BITS / 8);
      w0[k] = p[0];
      if (BITS == 8) w1[k] = p[1];
    }
  }
  const bool word_codes = !kv.qfmt || w == 0;
#pragma unroll
  for (int k = 0; k < kGatherPieces; k++) {
    if (!live[k]) continue;
    uint32_t c[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
      c[i] = !word_codes ? c4[k][i]
             : BITS == 4 ? (w0[k] >> (4 * i)) & kMask
                         : ((i < 4 ? w0[k] : w1[k]) >> (8 * (i & 3))) & kMask;
    typename E::T* o = static_cast<typename E::T*>(out) +
                       (static_cast<int64_t>(plane) * g.T + ti[k]) * g.D + d0[k];
    if constexpr (E::kBytes == 2) {
      uint32_t pk[4];
#pragma unroll
      for (int i = 0; i < 4; i++)
        pk[i] = static_cast<uint32_t>(E::from_f32(fmaf(sc[k], static_cast<float>(c[2 * i]), bi[k]))) |
                static_cast<uint32_t>(E::from_f32(fmaf(sc[k], static_cast<float>(c[2 * i + 1]), bi[k])))
                    << 16;
      *reinterpret_cast<uint4*>(o) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    } else {
      float f[8];
#pragma unroll
      for (int i = 0; i < 8; i++) f[i] = fmaf(sc[k], static_cast<float>(c[i]), bi[k]);
      reinterpret_cast<float4*>(o)[0] = make_float4(f[0], f[1], f[2], f[3]);
      reinterpret_cast<float4*>(o)[1] = make_float4(f[4], f[5], f[6], f[7]);
    }
  }
}

// Reference-layout affine rows -> paged chunks (inverse of the code gather).
template <int ESIZE, int BITS>
__global__ void __launch_bounds__(256) scatter_codes_kernel(ScatterCodesArgs a) {
  const int tpr = a.D / 8;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = gtid / tpr;  // (s, h, t)
  const int j = static_cast<int>(gtid % tpr);
  const int64_t total = static_cast<int64_t>(a.n_seqs) * a.H * a.T;
  if (row >= total) return;
  const int64_t t = row % a.T;
  const int64_t h = (row / a.T) % a.H;
  const int64_t s = row / (static_cast<int64_t>(a.T) * a.H);
  const RowDst& d = a.dst;
  const int32_t blk = d.table[s * d.table_stride + t / d.block_size];
  if (blk < 0) return;
  const int tib = static_cast<int>(t % d.block_size);
  uint8_t* chunk = d.base + static_cast<int64_t>(blk) * d.block_bytes + h * d.head_bytes;
  const uint32_t* w = a.wq + row * (a.D * BITS / 32);
  uint32_t code[8];
  if constexpr (BITS == 4) {
    const uint32_t x = w[j];
    for (int i = 0; i < 8; i++) code[i] = (x >> (4 * i)) & 15u;
  } else {
    const uint32_t x0 = w[2 * j], x1 = w[2 * j + 1];
    for (int i = 0; i < 4; i++) {
      code[i] = (x0 >> (8 * i)) & 255u;
      code[4 + i] = (x1 >> (8 * i)) & 255u;
    }
  }
  store_chunk_codes<BITS>(chunk, d, tib, j, a.D, code);
  if ((j * 8) % a.group == 0) {
    const int G = a.D / a.group;
    const int g = j * 8 / a.group;
    const uint8_t* sp = static_cast<const uint8_t*>(a.scales) + (row * G + g) * ESIZE;
    const uint8_t* bp = static_cast<const uint8_t*>(a.biases) + (row * G + g) * ESIZE;
    uint8_t* so = chunk + d.s_off + qsb_index(tib, d.is_v, g, 0, d.G, d.keys_only) * ESIZE;
    uint8_t* bo = chunk + d.s_off + qsb_index(tib, d.is_v, g, 1, d.G, d.keys_only) * ESIZE;
    for (int i = 0; i < ESIZE; i++) {
      so[i] = sp[i];
      bo[i] = bp[i];
    }
  }
}

// ------------------------------------------------------------ copy4d

template <typename U>
__global__ void __launch_bounds__(256) copy4d_kernel(const U* src, U* dst, int64_t n0, int64_t n1,
                                                     int64_t n2, int64_t n3, int64_t s0, int64_t s1,
                                                     int64_t s2, int64_t s3, int64_t d0, int64_t d1,
                                                     int64_t d2, int64_t d3) {
  const int64_t total = n0 * n1 * n2 * n3;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t i3 = i % n3;
    int64_t r = i / n3;
    int64_t i2 = r % n2;
    r /= n2;
    int64_t i1 = r % n1;
    int64_t i0 = r / n1;
    dst[i0 * d0 + i1 * d1 + i2 * d2 + i3 * d3] = src[i0 * s0 + i1 * s1 + i2 * s2 + i3 * s3];
  }
}

// Two strided 4-D copies of one element size in one launch (blockIdx.y
// picks the copy): a cache update writes its K and V tokens with one launch.
template <typename U>
__global__ void __launch_bounds__(256) copy4d_pair_kernel(Copy4D c0, Copy4D c1) {
  const Copy4D& c = blockIdx.y ? c1 : c0;
  const int64_t total = c.n[0] * c.n[1] * c.n[2] * c.n[3];
  const U* src = static_cast<const U*>(c.src);
  U* dst = static_cast<U*>(c.dst);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t i3 = i % c.n[3];
    int64_t r = i / c.n[3];
    int64_t i2 = r % c.n[2];
    r /= c.n[2];
    int64_t i1 = r % c.n[1];
    int64_t i0 = r / c.n[1];
    dst[i0 * c.d[0] + i1 * c.d[1] + i2 * c.d[2] + i3 * c.d[3]] =
        src[i0 * c.s[0] + i1 * c.s[1] + i2 * c.s[2] + i3 * c.s[3]];
  }
}

// Whole-block copy across all layers (copy-on-write, prefix store).  The
// (src, dst) pairs travel in the kernel arguments, so no device staging
// buffer has to outlive the launch.
__global__ void __launch_bounds__(256) copy_blocks_kernel(uint8_t* base, int64_t layer_bytes,
                                                          int64_t block_bytes, BlockPairs pairs) {
  const int pair = blockIdx.y;
  const int layer = blockIdx.z;
  const int64_t words = block_bytes / 16;
  const uint4* s = reinterpret_cast<const uint4*>(base + layer * layer_bytes +
                                                  static_cast<int64_t>(pairs.src[pair]) * block_bytes);
  uint4* d = reinterpret_cast<uint4*>(base + layer * layer_bytes +
                                      static_cast<int64_t>(pairs.dst[pair]) * block_bytes);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    d[i] = s[i];
}

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = v;
}

// ------------------------------------------------------------ synthetic

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

template <int DT>
__global__ void __launch_bounds__(256) fill_normal_kernel(void* data, int64_t n, uint64_t seed,
                                                          float std) {
  using E = Elem<DT>;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const uint64_t r = splitmix64(seed * 0x100000001B3ull + static_cast<uint64_t>(i));
    const float u1 = (static_cast<float>(r >> 40) + 1.0f) * (1.0f / 16777216.0f);
    const float u2 = static_cast<float>((r >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
    const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
    static_cast<typename E::T*>(data)[i] = E::from_f32(z * std);
  }
}

// ------------------------------------------------------------ attention
//
// Split-K decode attention, one workgroup (256 threads) per (partition,
// kv head, query row).  A workgroup walks its partition in tiles of 32
// tokens: 8 lanes per token form scores for the REP query heads that share
// the kv head (one K read serves all of them), one wave updates the running
// max / sum (online softmax, sdpa_vector.h:116-131), and each thread then
// accumulates P.V for one value dim.  Partials (unnormalised o, max, sum)
// are combined by attn_combine_kernel exactly as sdpa_vector_2pass_2 does
// (sdpa_vector.h:320-394); a single-partition launch normalises in place.
//
// QSEM selects the quantized-SDPA semantics of KVCache.swift:1909-1997:
// queries scaled in T, scores rounded to T, masked scores set to T's lowest
// value (so a fully masked row averages V).  Otherwise MLXFast semantics: queries scaled in
// fp32, masked keys skipped, an empty row yields zeros.
constexpr int kTile = 32;
constexpr int kMaxD = 256;

template <int DT, int BITS, int REP, bool QSEM>
__global__ void __launch_bounds__(256) attn_partial_kernel(AttnArgs a, int h_off, int rep_total) {
  using E = Elem<DT>;
  __shared__ float qs[REP][kMaxD];
  __shared__ float sc[REP][kTile];
  __shared__ float alpha_s[REP];
  __shared__ float red[256 * REP];

  const int tid = threadIdx.x;
  const int part = blockIdx.x;
  const int hk = blockIdx.y;
  const int64_t row = blockIdx.z;  // b * L + l
  const int64_t b = row / a.L;
  const int l = static_cast<int>(row % a.L);
  const int D = a.D, Dv = a.Dv;
  const int64_t T = a.kv.seq_lens ? a.kv.seq_lens[b] : a.kv.T;
  const int64_t t_begin = static_cast<int64_t>(part) * a.part_tokens;
  const int64_t t_end = min<int64_t>(T, t_begin + a.part_tokens);
  const float lowest = -E::kMax;
  const int group = a.group > 0 ? a.group : 64;

  // queries of the REP heads sharing kv head hk
  const float scale_t = QSEM ? round_to<DT>(a.scale) : a.scale;
  for (int i = tid; i < REP * D; i += 256) {
    const int r = i / D, d = i % D;
    const int h = hk * rep_total + h_off + r;
    const float qv = E::load(static_cast<const typename E::T*>(a.q) + b * a.q_sb + h * a.q_sh +
                             static_cast<int64_t>(l) * a.q_sl + d);
    qs[r][d] = QSEM ? round_to<DT>(qv * scale_t) : qv * scale_t;
  }

  // Phase-C thread layout: value dim `vd`, token subset `sub`.
  const int n_sub = max(1, 256 / Dv);
  const int vd = tid % Dv;
  const int sub = tid / Dv;
  const bool c_active = sub < n_sub && tid < n_sub * Dv;
  float o[REP];
#pragma unroll
  for (int r = 0; r < REP; r++) o[r] = 0.0f;
  float m_run = -3.402823466e38f, l_run = 0.0f;  // lanes r < REP of wave 0 own head r
  // an attention sink (MLXFast semantics only) is one more logit with a
  // zero value row, counted once per row (sdpa_vector.h:93-96, :257-260)
  if (!QSEM && a.sinks && part == 0 && tid < REP) {
    m_run = load_as<DT>(a.sinks, a.sinks_dtype, hk * rep_total + h_off + tid);
    l_run = 1.0f;
  }
  __syncthreads();

  for (int64_t t0 = t_begin; t0 < t_end; t0 += kTile) {
    // ---- phase A: scores
    {
      const int tt = tid / 8, lane = tid % 8;
      const int64_t t = t0 + tt;
      float acc[REP];
#pragma unroll
      for (int r = 0; r < REP; r++) acc[r] = 0.0f;
      if (t < t_end) {
        const TokLoc loc = locate(a.kv, b, t);
        for (int d = lane; d < D; d += 8) {
          const float kv = kv_at<DT, BITS>(a.kv, loc, hk, d, 0, group);
#pragma unroll
          for (int r = 0; r < REP; r++) acc[r] = fmaf(qs[r][d], kv, acc[r]);
        }
      }
#pragma unroll
      for (int r = 0; r < REP; r++) acc[r] = wave_sum(acc[r], 8);
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < REP; r++) {
          // quantized SDPA stores the scores in the dtype (quantizedMM
          // returns T, KVCache.swift:1945-1949) before the mask is applied
          float s = QSEM ? round_to<DT>(acc[r]) : acc[r];
          bool vis = t < t_end;
          if (vis && a.mask_mode != 0) {
            const int h = hk * rep_total + h_off + r;
            if (a.mask_mode == 1) {
              vis = t <= T - a.L + l;
            } else {
              const int64_t mo = b * a.m_sb + h * a.m_sh + l * a.m_sl + t * a.m_st;
              if (a.mask_mode == 2) {
                vis = static_cast<const uint8_t*>(a.mask)[mo] != 0;
              } else if (QSEM) {
                // scores (T) + mask: a T mask keeps the sum in T, an f32
                // mask promotes it to f32 (KVCache.swift:1963-1969)
                const float add = load_f32(a.mask, a.mask_dtype, mo);
                s = a.mask_dtype == DT ? round_to<DT>(s + add) : s + add;
              } else {
                // the mask in the query dtype; keys below its lowest finite
                // value are skipped (sdpa_vector.h:105-121)
                const float add = load_as<DT>(a.mask, a.mask_dtype, mo);
                vis = add >= -E::kMax;
                s += add;
              }
            }
            if (QSEM && !vis && t < t_end) {
              s = lowest;
              vis = true;
            }
          }
          sc[r][tt] = vis ? s : -INFINITY;
        }
      }
    }
    __syncthreads();
    // ---- phase B: online softmax update (wave 0, lane = token in tile)
    if (tid < 64) {
      const int tt = tid & 31;
#pragma unroll
      for (int r = 0; r < REP; r++) {
        const float s = sc[r][tt];
        float tmax = wave_max(tid < 32 ? s : -INFINITY, 64);
        const float m_old = __shfl(m_run, r, 64);
        const float m_new = fmaxf(m_old, tmax);
        const float p = (tid < 32 && s != -INFINITY) ? __expf(s - m_new) : 0.0f;
        const float psum = wave_sum(p, 64);
        const float al = __expf(m_old - m_new);
        if (tid < 32) sc[r][tt] = p;
        if (tid == r) {
          m_run = m_new;
          l_run = l_run * al + psum;
          alpha_s[r] = al;
        }
      }
    }
    __syncthreads();
    // ---- phase C: o = o * alpha + sum_t p_t v_t
    if (c_active) {
#pragma unroll
      for (int r = 0; r < REP; r++) o[r] *= alpha_s[r];
      for (int tt = sub; tt < kTile; tt += n_sub) {
        const int64_t t = t0 + tt;
        if (t >= t_end) break;
        const TokLoc loc = locate(a.kv, b, t);
        const float vv = kv_at<DT, BITS>(a.kv, loc, hk, vd, 1, group);
#pragma unroll
        for (int r = 0; r < REP; r++) o[r] = fmaf(sc[r][tt], vv, o[r]);
      }
    }
    __syncthreads();
  }

  // combine the token subsets of phase C
  if (c_active) {
#pragma unroll
    for (int r = 0; r < REP; r++) red[(r * n_sub + sub) * Dv + vd] = o[r];
  }
  if (tid < REP) {
    qs[tid][0] = m_run;  // reuse: per-head max / sum
    qs[tid][1] = l_run;
  }
  __syncthreads();
  for (int i = tid; i < REP * Dv; i += 256) {
    const int r = i / Dv, d = i % Dv;
    float acc = 0.0f;
    for (int s2 = 0; s2 < n_sub; s2++) acc += red[(r * n_sub + s2) * Dv + d];
    const float m = qs[r][0], lsum = qs[r][1];
    const int h = hk * rep_total + h_off + r;
    if (a.n_parts == 1) {
      const float v = lsum > 0.0f ? acc / lsum : 0.0f;
      static_cast<typename E::T*>(a.out)[b * a.o_sb + h * a.o_sh + static_cast<int64_t>(l) * a.o_sl +
                                         d] = E::from_f32(v);
    } else {
      const int64_t base = ((row * a.Hq + h) * a.n_parts + part);
      a.ws_o[base * Dv + d] = acc;
      if (d == 0) {
        a.ws_ml[base * 2] = m;
        a.ws_ml[base * 2 + 1] = lsum;
      }
    }
  }
}

// One wave per (row, head): lane l merges dims l, l + 64, .. (Dv <= 256).
// The (max, sum) pairs and partial rows of up to NP parts are loaded before
// any is used, so a merge costs one memory round trip per NP parts (NP = 2,
// 4 or 8, the smallest that holds the launch's parts, so few parts load no
// clamped duplicates).
template <int DT, int NP = 8>
__global__ void __launch_bounds__(256) attn_combine_kernel(AttnArgs a, int64_t n_rh) {
  using E = Elem<DT>;
  const int64_t rh = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);  // row * Hq + h
  if (rh >= n_rh) return;
  const int lane = threadIdx.x & 63;
  const int64_t row = rh / a.Hq;
  const int h = static_cast<int>(rh % a.Hq);
  const int64_t b = row / a.L;
  const int l = static_cast<int>(row % a.L);
  const float* ml = a.ws_ml + rh * a.n_parts * 2;
  const float* wo = a.ws_o + rh * a.n_parts * a.Dv;
  float M = -3.402823466e38f, den = 0.0f;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = 0; c < a.n_parts; c += NP) {
    float m[NP], ls[NP], v[NP][4];
#pragma unroll
    for (int j = 0; j < NP; j++) {
      const int p = min(c + j, a.n_parts - 1);  // (clamped slots are selected away)
      m[j] = ml[2 * p];
      ls[j] = ml[2 * p + 1];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int d = lane + 64 * i;
        v[j][i] = d < a.Dv ? wo[static_cast<int64_t>(p) * a.Dv + d] : 0.0f;
      }
    }
    float Mc = M;
#pragma unroll
    for (int j = 0; j < NP; j++)
      if (c + j < a.n_parts) Mc = fmaxf(Mc, m[j]);
    const float r = __expf(M - Mc);
    den *= r;
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] *= r;
    M = Mc;
#pragma unroll
    for (int j = 0; j < NP; j++) {
      if (c + j < a.n_parts) {
        const float w = __expf(m[j] - M);
        den += w * ls[j];
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = fmaf(w, v[j][i], acc[i]);
      }
    }
  }
  typename E::T* out = static_cast<typename E::T*>(a.out) + b * a.o_sb + h * a.o_sh +
                       static_cast<int64_t>(l) * a.o_sl;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int d = lane + 64 * i;
    if (d < a.Dv) out[d] = E::from_f32(den > 0.0f ? acc[i] / den : 0.0f);
  }
}

// The same merge for launches with few (row, head)s: one wave per (row,
// head, 64 dims), lane l merging dim 64 c + l, the (max, sum) pairs and
// partials of up to 32 parts loaded before any is used (the pairs are the
// same for the whole wave, so they load through the scalar path): four
// times the waves and one memory round trip per 32 parts.
template <int DT>
__global__ void __launch_bounds__(64) attn_combine_narrow_kernel(AttnArgs a, int64_t n_rh) {
  using E = Elem<DT>;
  const int nch = (a.Dv + 63) / 64;
  const int64_t rh = blockIdx.x / nch;  // row * Hq + h
  if (rh >= n_rh) return;
  const int d = 64 * static_cast<int>(blockIdx.x % nch) + threadIdx.x;
  const bool dv = d < a.Dv;
  const int64_t row = rh / a.Hq;
  const int h = static_cast<int>(rh % a.Hq);
  const int64_t b = row / a.L;
  const int l = static_cast<int>(row % a.L);
  const float* ml = a.ws_ml + rh * a.n_parts * 2;
  const float* wo = a.ws_o + rh * a.n_parts * a.Dv + (dv ? d : 0);
  float M = -3.402823466e38f, den = 0.0f, acc = 0.0f;
  for (int c = 0; c < a.n_parts; c += 32) {
    float m[32], ls[32], v[32];
#pragma unroll
    for (int j = 0; j < 32; j++) {
      const int p = min(c + j, a.n_parts - 1);  // (clamped slots are selected away)
      m[j] = ml[2 * p];
      ls[j] = ml[2 * p + 1];
      v[j] = wo[static_cast<int64_t>(p) * a.Dv];
    }
    float Mc = M;
#pragma unroll
    for (int j = 0; j < 32; j++)
      if (c + j < a.n_parts) Mc = fmaxf(Mc, m[j]);
    const float r = __expf(M - Mc);
    den *= r;
    acc *= r;
    M = Mc;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      if (c + j < a.n_parts) {
        const float w = __expf(m[j] - M);
        den += w * ls[j];
        acc = fmaf(w, v[j], acc);
      }
    }
  }
  if (dv) {
    typename E::T* out = static_cast<typename E::T*>(a.out) + b * a.o_sb + h * a.o_sh +
                         static_cast<int64_t>(l) * a.o_sl;
    out[d] = E::from_f32(den > 0.0f ? acc / den : 0.0f);
  }
}

// ------------------------------------------------------------ launchers

static inline unsigned blocks_for(int64_t threads) {
  return static_cast<unsigned>((threads + 255) / 256);
}

template <int DT>
static void quantize_dispatch(int bits, int group, int mode, const RowSrc& src, const RowDst& dst,
                              int64_t rows, int D, hipStream_t st) {
  const unsigned nb = blocks_for(rows * (D / 8));
#define VKV_Q(B, G, M) \
  hipLaunchKernelGGL((quantize_rows_kernel<DT, B, G, M>), dim3(nb), dim3(256), 0, st, src, dst, rows, D)
#define VKV_QM(B, G) \
  do { if (mode == 0) VKV_Q(B, G, 0); else VKV_Q(B, G, 1); } while (0)
#define VKV_QG(B)                               \
  do {                                          \
    if (group == 32) VKV_QM(B, 32);             \
    else if (group == 64) VKV_QM(B, 64);        \
    else if (group == 128) VKV_QM(B, 128);      \
    else throw Error("group_size must be 32, 64 or 128"); \
  } while (0)
  if (bits == 4) VKV_QG(4);
  else if (bits == 8) VKV_QG(8);
  else throw Error("bits must be 4 or 8");
#undef VKV_QG
#undef VKV_QM
#undef VKV_Q
}

void launch_quantize_rows(int dtype, int bits, int group, int mode, const RowSrc& src,
                          const RowDst& dst, int64_t rows, int D, hipStream_t st) {
  if (rows <= 0) return;
  VKV_CHECK(D % group == 0 && D % 8 == 0, "last dim must be a multiple of group_size");
  switch (dtype) {
    case kF32: quantize_dispatch<kF32>(bits, group, mode, src, dst, rows, D, st); break;
    case kF16: quantize_dispatch<kF16>(bits, group, mode, src, dst, rows, D, st); break;
    case kBF16: quantize_dispatch<kBF16>(bits, group, mode, src, dst, rows, D, st); break;
    default: throw Error("unsupported dtype");
  }
  VKV_HIP(hipGetLastError());
}

template <int DT>
static void append_dispatch(int bits, int group, const RowSrc& sk, const RowSrc& sv, const RowDst& dk,
                            const RowDst& dv, int64_t ntok, int H, int D, bool with_v, hipStream_t st) {
  const int hb = 256 / D;
  const dim3 grid(static_cast<unsigned>((ntok + 7) / 8), (H + hb - 1) / hb, with_v ? 2 : 1);
  const TimedLaunch tl = timing_prepare(kTimeAppend);
#define VKV_A(B, G)                                                                            \
  hipExtLaunchKernelGGL((append_affine_kernel<DT, B, G>), grid, dim3(256), 0, st, tl.start, tl.stop, \
                        0, sk, sv, dk, dv, ntok, H, D)
#define VKV_AG(B)                         \
  do {                                    \
    if (group == 32) VKV_A(B, 32);        \
    else if (group == 64) VKV_A(B, 64);   \
    else VKV_A(B, 128);                   \
  } while (0)
  if (bits == 4) VKV_AG(4);
  else VKV_AG(8);
#undef VKV_AG
#undef VKV_A
  VKV_HIP(hipGetLastError());
  timing_commit(tl);
}

bool append_affine_supported(int bits, int group, int D) {
  return (bits == 4 || bits == 8) && (group == 32 || group == 64 || group == 128) && D % group == 0 &&
         (D == 32 || D == 64 || D == 128 || D == 256);
}

void launch_append_affine(int dtype, int bits, int group, const RowSrc& sk, const RowSrc& sv,
                          const RowDst& dk, const RowDst& dv, int64_t ntok, int H, int D, bool with_v,
                          hipStream_t st) {
  if (ntok <= 0) return;
  VKV_CHECK(append_affine_supported(bits, group, D), "append_affine: unsupported geometry");
  switch (dtype) {
    case kF32: append_dispatch<kF32>(bits, group, sk, sv, dk, dv, ntok, H, D, with_v, st); break;
    case kF16: append_dispatch<kF16>(bits, group, sk, sv, dk, dv, ntok, H, D, with_v, st); break;
    case kBF16: append_dispatch<kBF16>(bits, group, sk, sv, dk, dv, ntok, H, D, with_v, st); break;
    default: throw Error("unsupported dtype");
  }
  VKV_HIP(hipGetLastError());
}

void launch_copy_rows(int dtype, int mode, const RowSrc& src, const RowDst& dst, int64_t rows,
                      int D, hipStream_t st) {
  if (rows <= 0) return;
  const unsigned nb = blocks_for(rows * ((D + 7) / 8));
  if (elem_bytes(dtype) == 2) {
    if (mode == 0) hipLaunchKernelGGL((copy_rows_kernel<2, 0>), dim3(nb), dim3(256), 0, st, src, dst, rows, D);
    else hipLaunchKernelGGL((copy_rows_kernel<2, 1>), dim3(nb), dim3(256), 0, st, src, dst, rows, D);
  } else {
    if (mode == 0) hipLaunchKernelGGL((copy_rows_kernel<4, 0>), dim3(nb), dim3(256), 0, st, src, dst, rows, D);
    else hipLaunchKernelGGL((copy_rows_kernel<4, 1>), dim3(nb), dim3(256), 0, st, src, dst, rows, D);
  }
  VKV_HIP(hipGetLastError());
}

void launch_dequantize(int dtype, int bits, int group, const uint32_t* wq, const void* scales,
                       const void* biases, void* out, int64_t rows, int D, hipStream_t st) {
  if (rows <= 0) return;
  VKV_CHECK(D % group == 0 && group % 8 == 0, "last dim must be a multiple of group_size");
  const unsigned nb = blocks_for(rows * (D / 8));
#define VKV_DQ(DT, B) \
  hipLaunchKernelGGL((dequantize_kernel<DT, B>), dim3(nb), dim3(256), 0, st, wq, scales, biases, out, rows, D, group)
#define VKV_DQB(DT) do { if (bits == 4) VKV_DQ(DT, 4); else if (bits == 8) VKV_DQ(DT, 8); else throw Error("bits must be 4 or 8"); } while (0)
  switch (dtype) {
    case kF32: VKV_DQB(kF32); break;
    case kF16: VKV_DQB(kF16); break;
    case kBF16: VKV_DQB(kBF16); break;
    default: throw Error("unsupported dtype");
  }
#undef VKV_DQB
#undef VKV_DQ
  VKV_HIP(hipGetLastError());
}

// Whether gather_dequant8_kernel's vector accesses fit the view.
static bool gather8_ok(const GatherArgs& g) {
  if (g.D % 8 || g.group % 8 || reinterpret_cast<uintptr_t>(g.out) % 16 ||
      reinterpret_cast<uintptr_t>(g.out_v) % 16)
    return false;
  const auto a4 = [](int64_t x) { return x % 4 == 0; };
  const KVSrc& kv = g.kv;
  if (kv.qfmt)
    return a4(static_cast<int64_t>(reinterpret_cast<uintptr_t>(kv.base))) && a4(kv.block_bytes) &&
           a4(kv.head_bytes) && a4(kv.kc_off) && a4(kv.vc_off);
  for (int which = 0; which < 2; which++) {
    if (which != g.which && !g.out_v) continue;
    const Comp& c = which ? kv.vc : kv.kc;
    if (!(a4(static_cast<int64_t>(reinterpret_cast<uintptr_t>(c.ptr))) && a4(c.sb) && a4(c.sh) &&
          a4(c.st)))
      return false;
  }
  return true;
}

template <int DT, int BITS>
static void gather_dispatch_kind(const GatherArgs& g, int out_kind, hipStream_t st) {
  const unsigned nb = blocks_for(static_cast<int64_t>(g.n_seqs) * g.H * g.T * ((g.D + 7) / 8));
  if (out_kind == 0) {
    if constexpr (BITS > 0) {
      const int64_t planes = static_cast<int64_t>(g.n_seqs) * g.H;
      const int64_t per_plane = static_cast<int64_t>(g.T) * (g.D / 8);
      if (gather8_ok(g) && planes > 0 && planes <= 65535 && per_plane > 0 && per_plane < (1 << 30)) {
        const dim3 grid(static_cast<unsigned>((per_plane + 256 * kGatherPieces - 1) / (256 * kGatherPieces)),
                        static_cast<unsigned>(planes), g.out_v ? 2u : 1u);
        hipLaunchKernelGGL((gather_dequant8_kernel<DT, BITS>), grid, dim3(256), 0, st, g);
        return;
      }
    }
    if (g.out_v) {  // element-wise kernel: one launch per matrix
      GatherArgs one = g;
      one.out_v = nullptr;
      for (int which = 0; which < 2; which++) {
        one.which = which;
        one.out = which ? g.out_v : g.out;
        hipLaunchKernelGGL((gather_kernel<DT, BITS, 0>), dim3(nb), dim3(256), 0, st, one);
      }
      return;
    }
    hipLaunchKernelGGL((gather_kernel<DT, BITS, 0>), dim3(nb), dim3(256), 0, st, g);
  } else {
    if constexpr (BITS > 0) {
      hipLaunchKernelGGL((gather_kernel<DT, BITS, 1>), dim3(nb), dim3(256), 0, st, g);
    } else {
      throw Error("code gather needs an affine view");
    }
  }
}

template <int DT>
static void gather_dispatch(const GatherArgs& g, int out_kind, hipStream_t st) {
  if (g.bits == 0) gather_dispatch_kind<DT, 0>(g, out_kind, st);
  else if (g.bits == 4) gather_dispatch_kind<DT, 4>(g, out_kind, st);
  else if (g.bits == 8) gather_dispatch_kind<DT, 8>(g, out_kind, st);
  else throw Error("bits must be 0, 4 or 8");
}

void launch_gather(const GatherArgs& g, int out_kind, hipStream_t st) {
  if (static_cast<int64_t>(g.n_seqs) * g.H * g.T == 0) return;
  switch (g.dtype) {
    case kF32: gather_dispatch<kF32>(g, out_kind, st); break;
    case kF16: gather_dispatch<kF16>(g, out_kind, st); break;
    case kBF16: gather_dispatch<kBF16>(g, out_kind, st); break;
    default: throw Error("unsupported dtype");
  }
  VKV_HIP(hipGetLastError());
}

void launch_scatter_codes(const ScatterCodesArgs& a, hipStream_t st) {
  const int64_t rows = static_cast<int64_t>(a.n_seqs) * a.H * a.T;
  if (rows <= 0) return;
  const unsigned nb = blocks_for(rows * (a.D / 8));
  const int es = elem_bytes(a.dtype);
  if (a.bits == 4 && es == 2) hipLaunchKernelGGL((scatter_codes_kernel<2, 4>), dim3(nb), dim3(256), 0, st, a);
  else if (a.bits == 4) hipLaunchKernelGGL((scatter_codes_kernel<4, 4>), dim3(nb), dim3(256), 0, st, a);
  else if (a.bits == 8 && es == 2) hipLaunchKernelGGL((scatter_codes_kernel<2, 8>), dim3(nb), dim3(256), 0, st, a);
  else if (a.bits == 8) hipLaunchKernelGGL((scatter_codes_kernel<4, 8>), dim3(nb), dim3(256), 0, st, a);
  else throw Error("bits must be 4 or 8");
  VKV_HIP(hipGetLastError());
}

void launch_copy4d(int esize, const void* src, const int64_t* n, const int64_t* s, void* dst,
                   const int64_t* d, hipStream_t st) {
  const int64_t total = n[0] * n[1] * n[2] * n[3];
  if (total <= 0) return;
  const unsigned nb = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65536));
  if (esize == 2) {
    hipLaunchKernelGGL((copy4d_kernel<uint16_t>), dim3(nb), dim3(256), 0, st,
                       static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), n[0], n[1],
                       n[2], n[3], s[0], s[1], s[2], s[3], d[0], d[1], d[2], d[3]);
  } else if (esize == 4) {
    hipLaunchKernelGGL((copy4d_kernel<uint32_t>), dim3(nb), dim3(256), 0, st,
                       static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), n[0], n[1],
                       n[2], n[3], s[0], s[1], s[2], s[3], d[0], d[1], d[2], d[3]);
  } else if (esize == 1) {
    hipLaunchKernelGGL((copy4d_kernel<uint8_t>), dim3(nb), dim3(256), 0, st,
                       static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), n[0], n[1],
                       n[2], n[3], s[0], s[1], s[2], s[3], d[0], d[1], d[2], d[3]);
  } else {
    throw Error("copy4d: element size must be 1, 2 or 4");
  }
  VKV_HIP(hipGetLastError());
}

void launch_copy4d_pair(int esize, const Copy4D& c0, const Copy4D& c1, hipStream_t st) {
  const int64_t t0 = c0.n[0] * c0.n[1] * c0.n[2] * c0.n[3];
  const int64_t t1 = c1.n[0] * c1.n[1] * c1.n[2] * c1.n[3];
  const int64_t total = std::max(t0, t1);
  if (total <= 0) return;
  const dim3 grid(static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65536)), 2);
  if (esize == 2)
    hipLaunchKernelGGL((copy4d_pair_kernel<uint16_t>), grid, dim3(256), 0, st, c0, c1);
  else if (esize == 4)
    hipLaunchKernelGGL((copy4d_pair_kernel<uint32_t>), grid, dim3(256), 0, st, c0, c1);
  else if (esize == 1)
    hipLaunchKernelGGL((copy4d_pair_kernel<uint8_t>), grid, dim3(256), 0, st, c0, c1);
  else
    throw Error("copy4d: element size must be 1, 2 or 4");
  VKV_HIP(hipGetLastError());
}

void launch_copy_blocks(const uint8_t* base, int64_t layer_bytes, int n_layers, int64_t block_bytes,
                        const int32_t* src, const int32_t* dst, int n, hipStream_t st) {
  VKV_CHECK(block_bytes % 16 == 0, "block bytes must be a multiple of 16");
  const unsigned gx = static_cast<unsigned>(std::min<int64_t>((block_bytes / 16 + 255) / 256, 64));
  for (int done = 0; done < n; done += BlockPairs::kMax) {
    BlockPairs bp;
    const int cnt = std::min(n - done, BlockPairs::kMax);
    for (int i = 0; i < cnt; i++) {
      bp.src[i] = src[done + i];
      bp.dst[i] = dst[done + i];
    }
    hipLaunchKernelGGL(copy_blocks_kernel, dim3(gx, cnt, n_layers), dim3(256), 0, st,
                       const_cast<uint8_t*>(base), layer_bytes, block_bytes, bp);
    VKV_HIP(hipGetLastError());
  }
}

void launch_fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t st) {
  if (n <= 0) return;
  const unsigned nb = static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 4096));
  hipLaunchKernelGGL(fill_i32_kernel, dim3(nb), dim3(256), 0, st, p, n, v);
  VKV_HIP(hipGetLastError());
}

void launch_fill_normal(int dtype, void* data, int64_t n, uint64_t seed, float std, hipStream_t st) {
  if (n <= 0) return;
  const unsigned nb = static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 1 << 16));
  switch (dtype) {
    case kF32: hipLaunchKernelGGL((fill_normal_kernel<kF32>), dim3(nb), dim3(256), 0, st, data, n, seed, std); break;
    case kF16: hipLaunchKernelGGL((fill_normal_kernel<kF16>), dim3(nb), dim3(256), 0, st, data, n, seed, std); break;
    case kBF16: hipLaunchKernelGGL((fill_normal_kernel<kBF16>), dim3(nb), dim3(256), 0, st, data, n, seed, std); break;
    default: throw Error("unsupported dtype");
  }
  VKV_HIP(hipGetLastError());
}

template <int DT, int BITS, bool QSEM>
static void attn_dispatch_rep(const AttnArgs& a, int64_t rows, hipStream_t st) {
  const int rep = a.Hq / a.Hkv;
  dim3 grid(a.n_parts, a.Hkv, static_cast<unsigned>(rows));
  int done = 0;
  while (done < rep) {
    const int left = rep - done;
    const int chunk = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
#define VKV_A(R) \
  hipLaunchKernelGGL((attn_partial_kernel<DT, BITS, R, QSEM>), grid, dim3(256), 0, st, a, done, rep)
    if (chunk == 8) VKV_A(8);
    else if (chunk == 4) VKV_A(4);
    else if (chunk == 2) VKV_A(2);
    else VKV_A(1);
#undef VKV_A
    done += chunk;
  }
  if (a.n_parts > 1) {
    const int64_t n_rh = rows * a.Hq;
    hipLaunchKernelGGL((attn_combine_kernel<DT>), dim3(static_cast<unsigned>((n_rh + 3) / 4)),
                       dim3(256), 0, st, a, n_rh);
  }
}

template <int DT>
static void attn_dispatch(int bits, bool qsem, const AttnArgs& a, int64_t rows, hipStream_t st) {
  if (bits == 0) {
    if (qsem) throw Error("quantized semantics need an affine cache");
    attn_dispatch_rep<DT, 0, false>(a, rows, st);
  } else if (bits == 4) {
    attn_dispatch_rep<DT, 4, true>(a, rows, st);
  } else if (bits == 8) {
    attn_dispatch_rep<DT, 8, true>(a, rows, st);
  } else {
    throw Error("bits must be 0, 4 or 8");
  }
}

void launch_attn_combine(int dtype, const AttnArgs& a, int64_t rows, hipStream_t st) {
  if (a.Dv > 256) throw Error("attention merge supports value dims up to 256");
  const int64_t n_rh = rows * a.Hq;
  const int64_t nch = (a.Dv + 63) / 64;
  if (n_rh * nch <= 2048) {
    // few (row, head)s: the narrow merge's waves fit the chip at once
    const dim3 g(static_cast<unsigned>(n_rh * nch));
    switch (dtype) {
      case kF32: hipLaunchKernelGGL((attn_combine_narrow_kernel<kF32>), g, dim3(64), 0, st, a, n_rh); break;
      case kF16: hipLaunchKernelGGL((attn_combine_narrow_kernel<kF16>), g, dim3(64), 0, st, a, n_rh); break;
      case kBF16: hipLaunchKernelGGL((attn_combine_narrow_kernel<kBF16>), g, dim3(64), 0, st, a, n_rh); break;
      default: throw Error("unsupported dtype");
    }
    VKV_HIP(hipGetLastError());
    return;
  }
  const dim3 grid(static_cast<unsigned>((n_rh + 3) / 4));
  const int np = a.n_parts <= 2 ? 2 : a.n_parts <= 4 ? 4 : 8;
#define VKV_C(T, N) hipLaunchKernelGGL((attn_combine_kernel<T, N>), grid, dim3(256), 0, st, a, n_rh)
#define VKV_CD(T)                   \
  do {                              \
    if (np == 2) VKV_C(T, 2);       \
    else if (np == 4) VKV_C(T, 4);  \
    else VKV_C(T, 8);               \
  } while (0)
  switch (dtype) {
    case kF32: VKV_CD(kF32); break;
    case kF16: VKV_CD(kF16); break;
    case kBF16: VKV_CD(kBF16); break;
    default: throw Error("unsupported dtype");
  }
#undef VKV_CD
#undef VKV_C
  VKV_HIP(hipGetLastError());
}

void launch_attention(int dtype, int bits, int group, bool quant_semantics,
                      const AttnArgs& a, int64_t rows, hipStream_t st) {
  if (rows <= 0) return;
  VKV_CHECK(a.D <= kMaxD && a.Dv <= kMaxD, "head dims above 256 are not supported here");
  VKV_CHECK(a.Hq % a.Hkv == 0, "query heads must be a multiple of kv heads");
  VKV_CHECK(bits == 0 || group == 32 || group == 64 || group == 128,
            "affine attention supports group_size 32, 64 or 128");
  VKV_CHECK(bits == 0 || a.group == group, "the attention arguments carry another group size");
  switch (dtype) {
    case kF32: attn_dispatch<kF32>(bits, quant_semantics, a, rows, st); break;
    case kF16: attn_dispatch<kF16>(bits, quant_semantics, a, rows, st); break;
    case kBF16: attn_dispatch<kBF16>(bits, quant_semantics, a, rows, st); break;
    default: throw Error("unsupported dtype");
  }
  VKV_HIP(hipGetLastError());
}

}  // namespace vkv
