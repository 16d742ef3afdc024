// vkv_mla.hip -- absorbed-latent MLA decode attention on gfx950 matrix
// cores: one shared latent head, many query heads.
//
// Semantics: GLM4MoELiteAttention's absorbed decode
// (Libraries/MLXLLM/Models/GLM4MOELite.swift:233-290) through
// mlaScaledDotProductAttention (Libraries/MLXLMCommon/AttentionUtils.swift:
// 43-75).  Every query head attends to the same cache entries; an entry is
// the 512-dim latent followed by the 64-dim rope key (576 dims) and the
// values are its first 512 dims.  Entries are stored 8-bit affine (group
// 64) and are dequantized to bf16 as the reference's dequantize produces
// them (fma(scale, code, bias) in fp32, rounded to bf16).  Scores and the
// probability-weighted sum accumulate in fp32 on the matrix cores; the
// probabilities enter the second contraction as bf16.
//
// Work layout.  A workgroup of 4 waves (one per SIMD) owns one (sequence,
// token split, group of 64*HB query heads).  Wave w owns 16*HB heads: it
// keeps their queries in registers as the B operand of S^T = K Q^T and
// their 16*HB x 512 fp32 output accumulators (64*HB MFMA tiles).  Per
// 32-token tile:
//   * the raw bytes (codes, then scale/bias) reach LDS by direct
//     global->LDS loads issued three tiles ahead into four staging buffers,
//     with the waits counted by hand (the compiler would otherwise wait for
//     every such load before any LDS read);
//   * the 256 threads dequantize the tile into a bf16 [32][576] LDS tile
//     (double buffered), 9 (token, 8-dim) pieces each;
//   * each wave computes its scores with 16x16x32 bf16 MFMAs (A = key rows,
//     B = its queries), so lane l holds head l % 16 for tokens
//     4*(l/16) + i and 16 + 4*(l/16) + i;
//   * online softmax with a lazily refreshed running max (refreshed only
//     when a score exceeds it by more than kTau, in log2 units);
//   * P V uses the same LDS tile as the value operand, read with the
//     transposing LDS load ds_read_b64_tr_b16: within each 16-lane group,
//     lane i receives element i % 4 of the 8 bytes that lane 4*e + i / 4
//     addressed, so pointing those lanes at 4 consecutive dims of tokens
//     Tb + e hands lane i the dim (i) of tokens Tb .. Tb + 3 -- exactly the
//     tokens its probability registers hold.
// Split partials (unnormalized output, running max, sum) are merged by
// mla_combine_kernel as sdpa_vector_2pass_2 merges them
// (Source/Cmlx/mlx-generated/metal/sdpa_vector.h:320-394).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <utility>

#include "vkv_device.h"
#include "vkv_internal.h"

namespace vkv {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;
typedef __attribute__((address_space(3))) i16x4_t l_i16x4_t;

constexpr int kDK = 576;                  // entry dims (latent + rope)
constexpr int kDV = 512;                  // value dims
constexpr int kTile = 32;                 // tokens per tile
constexpr int kRow = kDK + 8;             // bf16 per LDS key row (padded)
constexpr int kChunks = kDK / 32;         // K steps of the score MFMA
constexpr int kDB = kDV / 16;             // 16-dim output tiles
constexpr int kSbRow = (kDK / 64) * 4;    // (scale, bias) bytes per token
constexpr int kRawCodes = kTile * kDK;    // code bytes of a tile
constexpr int kRawBytes = kRawCodes + 2048;  // codes | scale/bias | landing pad
constexpr int kStages = 4;                // raw staging buffers
constexpr int kDmaPerWave = 5;            // 16-byte x 64-lane loads per wave per tile
constexpr int kPieces = kTile * (kDK / 8) / 256;  // dequant pieces per thread
constexpr int kMaxSplits = 64;
constexpr float kTau = 64.0f;    // headroom of the fixed running max (log2)
constexpr float kLog2e = 1.4426950408889634f;

static_assert(kPieces == 9, "piece mapping assumes 9 x 8 dims per thread");

template <int... Is, class F>
__device__ __forceinline__ void sfor_impl(std::integer_sequence<int, Is...>, F&& f) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void sfor(F&& f) {
  sfor_impl(std::make_integer_sequence<int, N>{}, f);
}

__device__ __forceinline__ f32x4_t mfma(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// 64 lanes x 16 bytes from global memory straight into LDS at lds + 16*lane.
// Issued as inline asm so that the compiler does not treat every later LDS
// read as waiting on it; the callers count vmcnt themselves.
__device__ __forceinline__ void dma16(const uint8_t* g, uint32_t lds) {
  // (one wait state between the M0 write and the load that reads it)
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}

template <int HB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
mla_kernel(const MlaArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t raw[kStages][kRawBytes];
  __shared__ __attribute__((aligned(16))) uint16_t kt[2][kTile * kRow];
  __shared__ __attribute__((aligned(16))) int restart_flag[1][4];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, n = lane & 15, g = lane >> 4;
  const int split = blockIdx.x, b = blockIdx.y;
  const int len = a.seq_lens ? a.seq_lens[b] : a.max_len;
  const int t0 = split * a.split_len;
  const int t1 = min(len, t0 + a.split_len);
  const int ntiles = t1 > t0 ? (t1 - t0 + kTile - 1) / kTile : 0;
  const int hw = blockIdx.z * (64 * HB) + wave * (16 * HB);  // first head of this wave
  const size_t slot = static_cast<size_t>(b) * a.n_splits + split;

  if (ntiles == 0) {
    if (a.n_splits == 1) {
      // an empty sequence yields zeros
      for (int hb = 0; hb < HB; hb++) {
        const int h = hw + 16 * hb + n;
        if (h < a.H)
          for (int d = g; d < kDV; d += 4) a.out[b * a.o_ss + h * a.o_sh + d] = 0;
      }
    } else if (g == 0) {
      for (int hb = 0; hb < HB; hb++) {
        const int h = hw + 16 * hb + n;
        if (h < a.H) {
          a.ws_ml[(slot * a.H + h) * 2] = -INFINITY;
          a.ws_ml[(slot * a.H + h) * 2 + 1] = 0.0f;
        }
      }
    }
    return;
  }

  // ---- raw tile loads: wave w issues loads w, w+4, ..., w+16 of the 20
  // (18 x 1 KB of codes, then the scale/bias bytes with a landing pad)
  auto issue = [&](int i) {
    const int ic = min(i, ntiles - 1);
    const int ts = t0 + kTile * ic;
    const int blk = ts / a.block_size, off = ts - blk * a.block_size;
    const uint8_t* chunk =
        a.base + static_cast<int64_t>(a.table[static_cast<int64_t>(b) * a.table_stride + blk]) *
                     a.block_bytes;
    const uint8_t* codes = chunk + off * kDK;
    const uint8_t* sb = chunk + a.sb_off + off * kSbRow;
    const uint32_t lds = lds_addr(&raw[i & (kStages - 1)][0]);
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int j = wave + 4 * r;
      dma16(codes + 1024 * j + 16 * lane, lds + 1024 * j);
    }
    if (wave < 2) {
      const int j = 16 + wave;
      dma16(codes + 1024 * j + 16 * lane, lds + 1024 * j);
    } else if (wave == 2) {
      dma16(sb + 16 * lane, lds + kRawCodes);
    } else {
      // 128 bytes remain; the other lanes re-read byte 0 into the pad
      dma16(sb + (lane < 8 ? 1024 + 16 * lane : 0), lds + kRawCodes + 1024);
    }
  };

  // ---- dequant pieces of this thread: token tk (fixed) and 8-dim storage
  // positions 8k + pp, k = 0..8.  Within 16 lanes: 4 tokens x 4 adjacent
  // positions, which keeps the 16-byte LDS stores free of bank conflicts.
  const int l16 = lane & 15, grp = lane >> 4;
  const int tk = 8 * wave + 4 * (grp & 1) + (l16 >> 2);
  const int pp = 4 * (grp >> 1) + (l16 & 3);
  struct Piece {
    u32x2_t c;
    uint32_t sb;
  };
  // dims 8q..8q+7 sit at storage position (q % 4) * 18 + q / 4 of a token row
  auto piece_q = [&](int k, int pp) {
    const int p = 8 * k + pp;
    const int run = (p >= 18) + (p >= 36) + (p >= 54);
    return 4 * (p - 18 * run) + run;
  };
  auto piece_read = [&](const uint8_t* r, int k, int pp) {
    Piece pc;
    pc.c = *reinterpret_cast<const u32x2_t*>(r + tk * kDK + 8 * (8 * k + pp));
    pc.sb = *reinterpret_cast<const uint32_t*>(r + kRawCodes + tk * kSbRow +
                                               4 * (piece_q(k, pp) >> 3));
    return pc;
  };
  auto piece_write = [&](const Piece& pc, uint16_t* dst, bool valid, int k, int pp) {
    const uint32_t sbw = valid ? pc.sb : 0u;  // tokens past the end become zeros
    const float s = __uint_as_float(sbw << 16), bb = __uint_as_float(sbw & 0xFFFF0000u);
    u32x4_t w;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t x = pc.c[h];
      w[2 * h] = pack_bf16(fmaf(s, static_cast<float>(x & 0xFF), bb),
                           fmaf(s, static_cast<float>((x >> 8) & 0xFF), bb));
      w[2 * h + 1] = pack_bf16(fmaf(s, static_cast<float>((x >> 16) & 0xFF), bb),
                               fmaf(s, static_cast<float>(x >> 24), bb));
    }
    *reinterpret_cast<u32x4_t*>(dst + 8 * piece_q(k, pp)) = w;
  };
  auto dequant_all = [&](int i) {
    const uint8_t* r = &raw[i & (kStages - 1)][0];
    uint16_t* dst = &kt[i & 1][tk * kRow];
    const bool valid = t0 + kTile * i + tk < t1;
    sfor<kPieces>([&](auto K) { piece_write(piece_read(r, K, pp), dst, valid, K, pp); });
  };

  // ---- queries (B operand of the score MFMA): head hw + 16 hb + n,
  // dims 32 c + 8 g .. +8
  u32x4_t qf[HB][kChunks];
#pragma unroll
  for (int hb = 0; hb < HB; hb++) {
    const int h = min(hw + 16 * hb + n, a.H - 1);
    const uint16_t* qp = a.q + b * a.q_ss + static_cast<int64_t>(h) * a.q_sh + 8 * g;
#pragma unroll
    for (int c = 0; c < kChunks; c++) qf[hb][c] = *(const g_u32x4_t*)(qp + 32 * c);
  }
  const float cl = a.scale * kLog2e;

  f32x4_t o[HB][kDB];
  float m_run[HB], l_run[HB], m_est[HB];
#pragma unroll
  for (int hb = 0; hb < HB; hb++) m_est[hb] = -INFINITY;

  // The running max starts at the first tile's max and is otherwise fixed:
  // probabilities up to 2^kTau are exact enough in fp32/bf16.  A score that
  // exceeds it by more than kTau makes the workgroup run the split again,
  // with m_est = the largest score of the whole first run, so the second
  // run never needs a third.  (The accumulators are never rescaled: a
  // rescale branch in the loop makes the compiler copy all of them on every
  // tile.)
  auto run = [&]() -> bool {
#pragma unroll
    for (int hb = 0; hb < HB; hb++) {
#pragma unroll
      for (int db = 0; db < kDB; db++) o[hb][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      m_run[hb] = m_est[hb];
      l_run[hb] = 0.f;
    }
    // prologue: tiles 0..2 in flight, tile 0 dequantized
    issue(0);
    issue(1);
    issue(2);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kDmaPerWave) : "memory");
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    dequant_all(0);

    int redo = 0;
    for (int i = 0; i < ntiles; i++) {
      issue(i + 3);
      // tile i+1's raw bytes are the oldest but two tiles of loads
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kDmaPerWave) : "memory");
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const uint16_t* K = &kt[i & 1][0];
      // scores S^T [32 tokens x 16*HB heads], with tile i+1's dequant
      // interleaved (piece k's LDS reads one step before its stores)
      // the piece offsets are recomputed each tile (a few VALU ops) rather
      // than held in 27 registers across the loop
      int ppv = pp;
      asm volatile("" : "+v"(ppv));
      const uint8_t* rn = &raw[(i + 1) & (kStages - 1)][0];
      uint16_t* dn = &kt[(i + 1) & 1][tk * kRow];
      const bool vn = t0 + kTile * (i + 1) + tk < t1;
      const uint16_t* kr0 = K + n * kRow + 8 * g;
      const uint16_t* kr1 = kr0 + 16 * kRow;
      f32x4_t s[2][HB];
#pragma unroll
      for (int tb = 0; tb < 2; tb++)
#pragma unroll
        for (int hb = 0; hb < HB; hb++) s[tb][hb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      u32x4_t ka[3][2];
      ka[0][0] = *reinterpret_cast<const u32x4_t*>(kr0);
      ka[0][1] = *reinterpret_cast<const u32x4_t*>(kr1);
      ka[1][0] = *reinterpret_cast<const u32x4_t*>(kr0 + 32);
      ka[1][1] = *reinterpret_cast<const u32x4_t*>(kr1 + 32);
      Piece pc[2];
      pc[0] = piece_read(rn, 0, ppv);
      sfor<kChunks>([&](auto C) {
        constexpr int c = decltype(C)::value;
        if constexpr (c + 2 < kChunks) {
          ka[(c + 2) % 3][0] = *reinterpret_cast<const u32x4_t*>(kr0 + 32 * (c + 2));
          ka[(c + 2) % 3][1] = *reinterpret_cast<const u32x4_t*>(kr1 + 32 * (c + 2));
        }
        if constexpr (c % 2 == 0 && c / 2 + 1 < kPieces)
          pc[(c / 2 + 1) & 1] = piece_read(rn, c / 2 + 1, ppv);
        if constexpr (c % 2 == 1) piece_write(pc[(c / 2) & 1], dn, vn, c / 2, ppv);
#pragma unroll
        for (int hb = 0; hb < HB; hb++) {
          s[0][hb] = mfma(ka[c % 3][0], qf[hb][c], s[0][hb]);
          s[1][hb] = mfma(ka[c % 3][1], qf[hb][c], s[1][hb]);
        }
        __builtin_amdgcn_sched_barrier(0);
      });

      // softmax (log2 domain) against the fixed running max
      const int rem = t1 - (t0 + kTile * i);
      float x[HB][2][4], mloc[HB];
      bool need = false;
#pragma unroll
      for (int hb = 0; hb < HB; hb++) {
        mloc[hb] = -INFINITY;
#pragma unroll
        for (int tb = 0; tb < 2; tb++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            float v = s[tb][hb][e] * cl;
            if (rem < kTile && 16 * tb + 4 * g + e >= rem) v = -INFINITY;
            x[hb][tb][e] = v;
            mloc[hb] = fmaxf(mloc[hb], v);
          }
        need |= mloc[hb] > m_run[hb] + kTau;
      }
      if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
        for (int hb = 0; hb < HB; hb++) {
          float mx = mloc[hb];
          mx = fmaxf(mx, __shfl_xor(mx, 16));
          mx = fmaxf(mx, __shfl_xor(mx, 32));
          m_est[hb] = fmaxf(m_est[hb], mx);
        }
        if (i == 0) {
          // nothing accumulated yet: take the max as is
#pragma unroll
          for (int hb = 0; hb < HB; hb++) m_run[hb] = m_est[hb];
        } else {
          redo = 1;
        }
      }
      u32x4_t pa[HB];
#pragma unroll
      for (int hb = 0; hb < HB; hb++) {
        float p[2][4];
        float ls = 0.f;
#pragma unroll
        for (int tb = 0; tb < 2; tb++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            p[tb][e] = fast_exp2(x[hb][tb][e] - m_run[hb]);
            ls += p[tb][e];
          }
        l_run[hb] += ls;
        pa[hb] = u32x4_t{pack_bf16(p[0][0], p[0][1]), pack_bf16(p[0][2], p[0][3]),
                         pack_bf16(p[1][0], p[1][1]), pack_bf16(p[1][2], p[1][3])};
      }

      // P V: value operand of dim 16 db + n, tokens 4g..4g+3 and
      // 16+4g..16+4g+3 (two transposing reads), four output tiles ahead
      const uint16_t* vr0 = K + (4 * g + (n >> 2)) * kRow + 4 * (n & 3);
      const uint16_t* vr1 = vr0 + 16 * kRow;
      auto vload = [&](int db) {
        const i16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((l_i16x4_t*)(vr0 + 16 * db));
        const i16x4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((l_i16x4_t*)(vr1 + 16 * db));
        const u32x2_t w0 = __builtin_bit_cast(u32x2_t, v0), w1 = __builtin_bit_cast(u32x2_t, v1);
        return u32x4_t{w0[0], w0[1], w1[0], w1[1]};
      };
      constexpr int kVA = 4;  // value operands in flight
      u32x4_t vb[kVA + 1];
      sfor<kVA>([&](auto D) { vb[D] = vload(D); });
      sfor<kDB>([&](auto D) {
        constexpr int db = decltype(D)::value;
        if constexpr (db + kVA < kDB) vb[(db + kVA) % (kVA + 1)] = vload(db + kVA);
#pragma unroll
        for (int hb = 0; hb < HB; hb++) o[hb][db] = mfma(pa[hb], vb[db % (kVA + 1)], o[hb][db]);
        __builtin_amdgcn_sched_barrier(0);
      });
    }
    // every raw-tile load has landed before the staging buffers are reused
    // or the workgroup ends; then agree on a second run
    if (lane == 0) restart_flag[0][wave] = redo;
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const u32x4_t f = *reinterpret_cast<const u32x4_t*>(&restart_flag[0][0]);
    const bool any = (f[0] | f[1] | f[2] | f[3]) != 0;
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    return any;
  };
  if (run()) run();

  // ---- finalize: lane (n, g) holds output rows (heads) 4g + e, dim 16 db + n
#pragma unroll
  for (int hb = 0; hb < HB; hb++) {
    float lt = l_run[hb];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);  // sum of head hw + 16 hb + n
    if (a.n_splits == 1) {
      const float inv = lt > 0.f ? 1.0f / lt : 0.f;
      float ir[4];
#pragma unroll
      for (int e = 0; e < 4; e++) ir[e] = __shfl(inv, 4 * g + e);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int h = hw + 16 * hb + 4 * g + e;
        if (h < a.H) {
          uint16_t* op = a.out + b * a.o_ss + static_cast<int64_t>(h) * a.o_sh + n;
#pragma unroll
          for (int db = 0; db < kDB; db++) op[16 * db] = f32_to_bf16(o[hb][db][e] * ir[e]);
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int h = hw + 16 * hb + 4 * g + e;
        if (h < a.H) {
          float* op = a.ws_o + (slot * a.H + h) * kDV + n;
#pragma unroll
          for (int db = 0; db < kDB; db++) op[16 * db] = o[hb][db][e];
        }
      }
      const int h = hw + 16 * hb + n;
      if (g == 0 && h < a.H) {
        a.ws_ml[(slot * a.H + h) * 2] = m_run[hb];
        a.ws_ml[(slot * a.H + h) * 2 + 1] = lt;
      }
    }
  }
}

// Merge of the split partials of one (sequence, head): 128 threads x 4 dims.
__global__ void __launch_bounds__(128) mla_combine_kernel(const MlaArgs a) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int d = 4 * threadIdx.x;
  const size_t s0 = static_cast<size_t>(b) * a.n_splits;
  float M = -INFINITY;
  for (int s = 0; s < a.n_splits; s++) {
    const float* ml = a.ws_ml + ((s0 + s) * a.H + h) * 2;
    if (ml[1] > 0.f) M = fmaxf(M, ml[0]);
  }
  float den = 0.f;
  f32x4_t acc{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < a.n_splits; s++) {
    const float* ml = a.ws_ml + ((s0 + s) * a.H + h) * 2;
    const float l = ml[1];
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(a.ws_o + ((s0 + s) * a.H + h) * kDV + d);
    const float w = l > 0.f ? fast_exp2(ml[0] - M) : 0.f;
    den += w * l;
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] = l > 0.f ? acc[e] + w * v[e] : acc[e];
  }
  const float inv = den > 0.f ? 1.0f / den : 0.f;
  uint16_t* op = a.out + b * a.o_ss + static_cast<int64_t>(h) * a.o_sh + d;
#pragma unroll
  for (int e = 0; e < 4; e++) op[e] = f32_to_bf16(acc[e] * inv);
}

int device_cus() {
  static int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 256;
    return std::max(1, n);
  }();
  return cus;
}

}  // namespace

bool mla_supported(int dtype, int bits, int group, int head_dim, int v_head_dim, int n_kv_heads,
                   int block_size) {
  return dtype == kBF16 && bits == 8 && group == 64 && head_dim == kDK && v_head_dim == kDV &&
         n_kv_heads == 1 && block_size > 0 && block_size % kTile == 0;
}

size_t mla_plan(MlaArgs& a, int want) {
  const int hb = a.H > 64 ? 2 : 1;
  const int groups = (a.H + 64 * hb - 1) / (64 * hb);
  const int max_tiles = std::max(1, (a.max_len + kTile - 1) / kTile);
  int splits = want > 0 ? want
                        : (device_cus() + a.n_seqs * groups - 1) / std::max(1, a.n_seqs * groups);
  splits = std::max(1, std::min({splits, max_tiles, kMaxSplits}));
  const int per = (max_tiles + splits - 1) / splits;  // tiles per split
  a.split_len = per * kTile;
  a.n_splits = (max_tiles + per - 1) / per;
  if (a.n_splits == 1) return 0;
  return static_cast<size_t>(a.n_seqs) * a.n_splits * a.H * (kDV + 2);
}

void launch_mla(const MlaArgs& a0, hipStream_t st) {
  MlaArgs a = a0;
  if (a.n_splits > 1) a.ws_ml = a.ws_o + static_cast<size_t>(a.n_seqs) * a.n_splits * a.H * kDV;
  const int hb = a.H > 64 ? 2 : 1;
  const dim3 grid(a.n_splits, a.n_seqs, (a.H + 64 * hb - 1) / (64 * hb));
  if (hb == 2)
    hipLaunchKernelGGL(mla_kernel<2>, grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(mla_kernel<1>, grid, dim3(256), 0, st, a);
  VKV_HIP(hipGetLastError());
  if (a.n_splits > 1) {
    hipLaunchKernelGGL(mla_combine_kernel, dim3(a.H, a.n_seqs), dim3(128), 0, st, a);
    VKV_HIP(hipGetLastError());
  }
}

}  // namespace vkv
