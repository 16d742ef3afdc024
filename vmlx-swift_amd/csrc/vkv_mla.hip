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
// token split, group of 64*HB query heads); per 32-token tile:
//   * every thread loads 9 (token, 8-dim) pieces of raw codes and their
//     scale/bias straight into registers one tile ahead, and dequantizes
//     them into a bf16 [32][576] LDS key tile (double buffered);
//   * wave w computes the scores of its 16*HB heads, S^T = K Q^T, with
//     16x16x32 bf16 MFMAs (A = key rows from LDS, B = its queries, held in
//     registers), so lane l holds head l % 16 for tokens 4*(l/16) + i and
//     16 + 4*(l/16) + i; softmax against a fixed running max; the
//     probabilities of all heads meet in an LDS tile;
//   * wave w then accumulates output dims [128w, 128w + 128) of every head
//     of the group: A = probabilities from LDS, B = the key tile read with
//     the transposing LDS load ds_read_b64_tr_b16 (within each 16-lane
//     group, lane i receives element i % 4 of the 8 bytes that lane
//     4*e + i / 4 addressed, so pointing those lanes at 4 consecutive dims
//     of tokens Tb + e hands lane i dim i of tokens Tb .. Tb + 3 -- exactly
//     the tokens the probability operand pairs it with), while the next
//     tile is dequantized.
// Each key element is read from LDS once per wave for the scores and once
// per workgroup for the values, which keeps the LDS below the matrix cores'
// rate.  Split partials (o / l in bf16, running max, sum) are merged by
// mla_combine_kernel as sdpa_vector_2pass_2 merges them
// (Source/Cmlx/mlx-generated/metal/sdpa_vector.h:320-394).
//
// LDS key tile layout.  Row t (token) holds the 72 8-dim pieces in the
// chunk format's storage order (piece q at position p = (q % 4) * 18 +
// q / 4, i.e. run p / 18 = q % 4, index p % 18 = q / 4), 16 bytes each, at
// slot 24 * (p / 18) + p % 18 + (t % 16) of a 112-slot (1792-byte) row.
// The score operand (16 rows, one position) and the transposing reads (8
// rows, two pieces one run apart) land on distinct banks; the dequant
// stores (tokens t and t + 8, 8 adjacent positions) do too except where
// the 8 positions cross a run.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <utility>

#include "vkv_device.h"
#include <hip/hip_ext.h>

#include "vkv_internal.h"

// Scale/bias row of zeros, read in place of the rows of tokens past the end.
__device__ uint32_t vkv_mla_zero_sb[16];

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
typedef __attribute__((address_space(1))) const u32x2_t g_u32x2_t;
typedef __attribute__((address_space(1))) const uint32_t g_u32_t;
typedef __attribute__((address_space(3))) i16x4_t l_i16x4_t;

constexpr int kDK = 576;                  // entry dims (latent + rope)
constexpr int kDV = 512;                  // value dims
constexpr int kTile = 32;                 // tokens per tile
constexpr int kPos = kDK / 8;             // 8-dim pieces per entry
constexpr int kRowB = 112 * 16;           // bytes per LDS key row (112 slots)
constexpr int kChunks = kDK / 32;         // K steps of the score MFMA
constexpr int kDW = kDV / 4;              // output dims per wave
constexpr int kDBW = kDW / 16;            // 16-dim output tiles per wave
constexpr int kPRow = 40;                 // bf16 per probability row (32 + pad)
constexpr int kSbRow = (kDK / 64) * 4;    // (scale, bias) bytes per token
constexpr int kPieces = kTile * kPos / 256;  // dequant pieces per thread
constexpr int kQReg = 16;                 // query chunks held in registers (rest in LDS)
constexpr int kQL = kChunks - kQReg;      // query chunks read from LDS
constexpr int kMaxSplits = 64;
constexpr float kTau = 64.0f;    // headroom of the fixed running max (log2)
constexpr float kLog2e = 1.4426950408889634f;

static_assert(kPieces == 9, "piece mapping assumes 9 x 8 dims per thread");

// Storage position p of a token row holds dims 8q..8q+7 with
// q = 4 * (p % 18) + p / 18; their scale/bias group is q / 8.
constexpr int pos_group(int p) { return (4 * (p % 18) + p / 18) / 8; }
// Piece k of a thread covers positions 8k + pb, pb = 0..7: 4-bit fields of
// the group and 2-bit fields of the run p / 18, indexed by pb.
constexpr uint32_t piece_groups(int k) {
  uint32_t v = 0;
  for (int pb = 0; pb < 8; pb++) v |= static_cast<uint32_t>(pos_group(8 * k + pb)) << (4 * pb);
  return v;
}
constexpr uint32_t piece_runs(int k) {
  uint32_t v = 0;
  for (int pb = 0; pb < 8; pb++) v |= static_cast<uint32_t>((8 * k + pb) / 18) << (2 * pb);
  return v;
}

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
// LDS pointer (address space 3, so accesses are ds_* instructions) from an
// LDS byte address.
template <class T>
__device__ __forceinline__ __attribute__((address_space(3))) T* lds_ptr(uint32_t a) {
  return reinterpret_cast<__attribute__((address_space(3))) T*>(static_cast<uintptr_t>(a));
}
// A uniform 32-bit word through the scalar path (a vector load would make
// the compiler wait for every load in flight before using it).
__device__ __forceinline__ int32_t scalar_load(const int32_t* p, int64_t i) {
  return *(reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(
               reinterpret_cast<uintptr_t>(p)) +
           i);
}

template <int HB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
mla_kernel(const MlaArgs a) {
  constexpr int kHeads = 64 * HB;     // query heads of the workgroup
  constexpr int kHB = kHeads / 16;    // their 16-head blocks
  __shared__ __attribute__((aligned(16))) uint8_t kt[2][kTile * kRowB];
  __shared__ __attribute__((aligned(16))) uint16_t pl[kHeads][kPRow];
  __shared__ __attribute__((aligned(16))) float lsh[kHeads];
  __shared__ __attribute__((aligned(16))) int restart_flag[4];
  // query chunks kQReg.. of every head: [chunk][head][32 dims + 8 pad]
  __shared__ __attribute__((aligned(16))) uint16_t qsh[kQL > 0 ? kQL : 1][kHeads][40];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, n = lane & 15, g = lane >> 4;
  const int split = blockIdx.x, b = blockIdx.y;
  const int len = a.seq_lens ? scalar_load(a.seq_lens, b) : a.max_len;
  const int t0 = split * a.split_len;
  const int t1 = min(len, t0 + a.split_len);
  const int ntiles = t1 > t0 ? (t1 - t0 + kTile - 1) / kTile : 0;
  const int hg0 = blockIdx.z * kHeads;        // first head of the workgroup
  const int hw = hg0 + wave * (16 * HB);      // first head this wave scores
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

  // ---- raw pieces of this thread: token tk, storage positions 8k + pb
  // (k = 0..8).  A 16-lane group covers tokens t and t + 8 x 8 adjacent
  // positions (64 contiguous bytes of each token row).  The loads go to
  // registers one tile ahead; tokens past the end read the zero
  // scale/bias row, so they dequantize to zeros.  ob is an opaque zero
  // (one per tile) that keeps the per-piece offsets from being hoisted out
  // of the tile loop into registers.
  const int l16 = tid & 15, pb = l16 & 7, grp = tid >> 4;
  const int tk = (grp & 7) + 16 * (grp >> 3) + 8 * (l16 >> 3);
  struct Raw {
    u32x2_t c[kPieces];
    uint32_t sb[kPieces];
  };
  auto load_raw_piece = [&](int i, int ob, int k, Raw& r) __attribute__((always_inline)) {
    const int ts = t0 + kTile * min(i, ntiles - 1);
    const int blk = ts / a.block_size, off = ts - blk * a.block_size;
    const uint8_t* chunk =
        a.base + static_cast<int64_t>(scalar_load(a.table, static_cast<int64_t>(b) * a.table_stride +
                                                                blk)) *
                     a.block_bytes;
    const int pbo = pb + ob;
    const uint8_t* cp = chunk + (off + tk) * kDK + 8 * pbo;
    const bool valid = t0 + kTile * i + tk < t1;
    const uint8_t* sp = valid ? chunk + a.sb_off + (off + tk) * kSbRow
                              : reinterpret_cast<const uint8_t*>(vkv_mla_zero_sb);
    r.c[k] = *(const g_u32x2_t*)(cp + 64 * k);
    r.sb[k] = *(const g_u32_t*)(sp + 4 * ((piece_groups(k) >> (4 * pbo)) & 15));
  };
  auto dequant_piece = [&](const Raw& r, int i, int ob, int k) __attribute__((always_inline)) {
    const int pbo = pb + ob;
    uint8_t* dst = &kt[i & 1][tk * kRowB + 16 * (pbo + (tk & 15))];
    const uint32_t sbw = r.sb[k];
    const float s = __uint_as_float(sbw << 16), bb = __uint_as_float(sbw & 0xFFFF0000u);
    u32x4_t w;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t x = r.c[k][h];
      w[2 * h] = pack_bf16(fmaf(s, static_cast<float>(x & 0xFF), bb),
                           fmaf(s, static_cast<float>((x >> 8) & 0xFF), bb));
      w[2 * h + 1] = pack_bf16(fmaf(s, static_cast<float>((x >> 16) & 0xFF), bb),
                               fmaf(s, static_cast<float>(x >> 24), bb));
    }
    // slot p + 6 * (p / 18) + (tk % 16), p = 8k + pb
    *reinterpret_cast<u32x4_t*>(dst + 128 * k + 96 * ((piece_runs(k) >> (2 * pbo)) & 3)) = w;
  };

  // ---- queries (B operand of the score MFMA): head hw + 16 hb + n,
  // dims 32 c + 8 g .. +8
  u32x4_t qf[HB][kQReg];
#pragma unroll
  for (int hb = 0; hb < HB; hb++) {
    const int h = min(hw + 16 * hb + n, a.H - 1);
    const uint16_t* qp = a.q + b * a.q_ss + static_cast<int64_t>(h) * a.q_sh + 8 * g;
#pragma unroll
    for (int c = 0; c < kQReg; c++) qf[hb][c] = *(const g_u32x4_t*)(qp + 32 * c);
#pragma unroll
    for (int c = kQReg; c < kChunks; c++)
      *reinterpret_cast<u32x4_t*>(&qsh[c - kQReg][wave * 16 * HB + 16 * hb + n][8 * g]) =
          *(const g_u32x4_t*)(qp + 32 * c);
  }
  const float cl = a.scale * kLog2e;

  f32x4_t o[kHB][kDBW];  // output rows (heads) 16 hb' + 4g + e, dims 128 wave + 16 db' + n
  float m_run[HB], l_run[HB], m_est[HB];
#pragma unroll
  for (int hb = 0; hb < HB; hb++) m_est[hb] = -INFINITY;

  // ---- scores S^T [32 tokens x 16*HB heads] of tile i.  Piece position
  // 18g + c (dims 32c + 8g..) of row t sits at slot 24g + c + (t % 16).
  f32x4_t s[2][HB];
  auto qk = [&](int i, int ob, Raw& r) __attribute__((always_inline)) {
    const uint32_t k0 =
        lds_addr(&kt[i & 1][0]) + n * kRowB + 16 * (24 * g + n) + ob;
#pragma unroll
    for (int tb = 0; tb < 2; tb++)
#pragma unroll
      for (int hb = 0; hb < HB; hb++) s[tb][hb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    u32x4_t ka[2][2];
    ka[0][0] = *lds_ptr<const u32x4_t>(k0);
    ka[0][1] = *lds_ptr<const u32x4_t>(k0 + 16 * kRowB);
    sfor<kChunks>([&](auto C) {
      constexpr int c = decltype(C)::value;
      if constexpr (c + 1 < kChunks) {
        ka[(c + 1) & 1][0] = *lds_ptr<const u32x4_t>(k0 + 16 * (c + 1));
        ka[(c + 1) & 1][1] = *lds_ptr<const u32x4_t>(k0 + 16 * kRowB + 16 * (c + 1));
      }
      // tile i+1's dequant (from registers), each piece followed by tile
      // i+2's load into the registers it frees: one piece every other step
      if constexpr (c % 2 == 1) {
        dequant_piece(r, i + 1, ob, c / 2);
        load_raw_piece(i + 2, ob, c / 2, r);
      }
#pragma unroll
      for (int hb = 0; hb < HB; hb++) {
        u32x4_t qb;
        if constexpr (c < kQReg)
          qb = qf[hb][c];
        else
          qb = *reinterpret_cast<const u32x4_t*>(
              &qsh[c - kQReg][wave * 16 * HB + 16 * hb + n][8 * g + ob]);
        s[0][hb] = mfma(ka[c & 1][0], qb, s[0][hb]);
        s[1][hb] = mfma(ka[c & 1][1], qb, s[1][hb]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // ---- softmax of tile i against the fixed running max: mask the tokens
  // past the end (last tile only), check the scores, write the
  // probabilities (bf16, the P.V operand layout: head row, tokens 4g..4g+3
  // then 16+4g..16+4g+3) to the workgroup's probability tile.  Returns
  // true when the split must be run again.
  auto softmax = [&](int i, int ob) __attribute__((always_inline)) -> bool {
    const int rem = t1 - (t0 + kTile * i);
    if (rem < kTile) {
      asm volatile("");  // keep this a branch: the mask is for one tile in many
      const int r4 = rem - 4 * g - ob;
#pragma unroll
      for (int tb = 0; tb < 2; tb++)
#pragma unroll
        for (int hb = 0; hb < HB; hb++)
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (16 * tb + e >= r4) s[tb][hb][e] = -INFINITY;
    }
    float mloc[HB];
    bool need = false;
#pragma unroll
    for (int hb = 0; hb < HB; hb++) {
      // scale > 0, so the largest score maps to the largest logit
      mloc[hb] = fmaxf(fmaxf(fmaxf(s[0][hb][0], s[0][hb][1]), fmaxf(s[0][hb][2], s[0][hb][3])),
                       fmaxf(fmaxf(s[1][hb][0], s[1][hb][1]), fmaxf(s[1][hb][2], s[1][hb][3]))) *
                 cl;
      need |= mloc[hb] > m_run[hb] + kTau;
    }
    bool redo = false;
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
        redo = true;
      }
    }
#pragma unroll
    for (int hb = 0; hb < HB; hb++) {
      float p[2][4];
#pragma unroll
      for (int tb = 0; tb < 2; tb++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          p[tb][e] = fast_exp2(fmaf(s[tb][hb][e], cl, -m_run[hb]));
          l_run[hb] += p[tb][e];
        }
      *reinterpret_cast<u32x4_t*>(&pl[wave * 16 * HB + 16 * hb + n][8 * g + ob]) =
          u32x4_t{pack_bf16(p[0][0], p[0][1]), pack_bf16(p[0][2], p[0][3]),
                  pack_bf16(p[1][0], p[1][1]), pack_bf16(p[1][2], p[1][3])};
    }
    return redo;
  };

  // ---- P V of tile i for output dims [128 wave, 128 wave + 128) of all the
  // workgroup's heads, with tile i+1's dequant (from registers) and tile
  // i+2's raw loads interleaved.  Value operand of dim d = 128 wave +
  // 16 db' + n: the pieces of dims d - (d % 8) live at storage position
  // p = 18 (2 (db' % 2) + e) + 4 wave + db' / 2 (e = (n % 4) / 2), slot
  // 24 (2 (db' % 2) + e) + 4 wave + db' / 2 + (row % 16).
  auto pv = [&](int i, int ob) __attribute__((always_inline)) {
    const int row = 4 * g + (n >> 2), e = (n & 3) >> 1;
    const uint32_t v0 = lds_addr(&kt[i & 1][0]) + row * kRowB +
                        16 * (24 * e + 4 * wave + (row & 15)) + 8 * (n & 1) + ob;
    const uint16_t* prow = &pl[n][8 * g + ob];
    // two halves of 4 output tiles: value operands of a half held, the
    // probability operands streamed (read twice)
    constexpr int kHalf = kDBW / 2;
    sfor<2>([&](auto HH) {
      constexpr int half = decltype(HH)::value;
      u32x4_t vb[kHalf];
      sfor<kHalf>([&](auto D) {
        constexpr int db = half * kHalf + decltype(D)::value;
        constexpr int off = 16 * (48 * (db & 1) + (db >> 1));
        const i16x4_t x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_ptr<i16x4_t>(v0 + off));
        const i16x4_t x1 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_ptr<i16x4_t>(v0 + off + 16 * kRowB));
        const u32x2_t w0 = __builtin_bit_cast(u32x2_t, x0), w1 = __builtin_bit_cast(u32x2_t, x1);
        vb[decltype(D)::value] = u32x4_t{w0[0], w0[1], w1[0], w1[1]};
      });
      u32x4_t pa[2];
      pa[0] = *reinterpret_cast<const u32x4_t*>(prow);
      sfor<kHB>([&](auto H) {
        constexpr int hb = decltype(H)::value;
        if constexpr (hb + 1 < kHB)
          pa[(hb + 1) & 1] = *reinterpret_cast<const u32x4_t*>(prow + 16 * kPRow * (hb + 1));
#pragma unroll
        for (int d = 0; d < kHalf; d++)
          o[hb][half * kHalf + d] = mfma(pa[hb & 1], vb[d], o[hb][half * kHalf + d]);
        __builtin_amdgcn_sched_barrier(0);
      });
    });
  };

  // The running max starts at the first tile's max and is otherwise fixed:
  // probabilities up to 2^kTau are exact enough in fp32/bf16.  A score that
  // exceeds it by more than kTau makes the workgroup run the split again,
  // with m_est = the largest score of the whole first run, so the second
  // run never needs a third.  (The accumulators are never rescaled: a
  // rescale branch in the loop makes the compiler copy all of them on every
  // tile.)  Two barriers per tile: before the scores (key tile i complete,
  // probability tile free) and before P.V (probabilities complete).
  auto run = [&]() __attribute__((always_inline)) -> bool {
#pragma unroll
    for (int hb = 0; hb < kHB; hb++)
#pragma unroll
      for (int db = 0; db < kDBW; db++) o[hb][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int hb = 0; hb < HB; hb++) {
      m_run[hb] = m_est[hb];
      l_run[hb] = 0.f;
    }
    Raw r;
    sfor<kPieces>([&](auto K) { load_raw_piece(0, 0, K, r); });
    sfor<kPieces>([&](auto K) {
      dequant_piece(r, 0, 0, K);
      load_raw_piece(1, 0, K, r);
    });
    bool redo = false;
    for (int i = 0; i < ntiles; i++) {
      int ob = 0;
      asm volatile("" : "+v"(ob));
      __syncthreads();
      qk(i, ob, r);
      redo |= softmax(i, ob);
      __syncthreads();
      pv(i, ob);
    }
    // total sums of this wave's heads for the normalization by all waves,
    // and agreement on a second run
#pragma unroll
    for (int hb = 0; hb < HB; hb++) {
      float lt = l_run[hb];
      lt += __shfl_xor(lt, 16);
      lt += __shfl_xor(lt, 32);
      l_run[hb] = lt;
      if (g == 0) lsh[wave * 16 * HB + 16 * hb + n] = lt;
    }
    if (lane == 0) restart_flag[wave] = redo ? 1 : 0;
    __syncthreads();
    const u32x4_t f = *reinterpret_cast<const u32x4_t*>(&restart_flag[0]);
    const bool any = (f[0] | f[1] | f[2] | f[3]) != 0;
    __syncthreads();
    return any;
  };
  // (one copy of the tile loop: a second inlined copy would keep values of
  // both alive and spill)
#pragma nounroll
  for (int attempt = 0; attempt < 2; attempt++)
    if (!run()) break;

  // ---- finalize: lane (n, g) holds output rows (heads) 16 hb' + 4g + e,
  // dims 128 wave + 16 db' + n.  Whole sequence: the output; a split: its
  // normalized partial (bf16), and (max, sum) from the heads' score wave.
  uint16_t* dst = a.n_splits == 1 ? a.out : a.ws_o;
  const int64_t dss = a.n_splits == 1 ? a.o_ss : static_cast<int64_t>(a.H) * kDV;
  const int64_t dsh = a.n_splits == 1 ? a.o_sh : kDV;
  const int64_t drow = a.n_splits == 1 ? b : static_cast<int64_t>(slot);
#pragma unroll
  for (int hb = 0; hb < kHB; hb++) {
    const f32x4_t lt = *reinterpret_cast<const f32x4_t*>(&lsh[16 * hb + 4 * g]);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int h = hg0 + 16 * hb + 4 * g + e;
      const float inv = lt[e] > 0.f ? 1.0f / lt[e] : 0.f;
      if (h < a.H) {
        uint16_t* op = dst + drow * dss + static_cast<int64_t>(h) * dsh + kDW * wave + n;
#pragma unroll
        for (int db = 0; db < kDBW; db++) op[16 * db] = f32_to_bf16(o[hb][db][e] * inv);
      }
    }
  }
  if (a.n_splits > 1 && g == 0) {
#pragma unroll
    for (int hb = 0; hb < HB; hb++) {
      const int h = hw + 16 * hb + n;
      if (h < a.H) {
        a.ws_ml[(slot * a.H + h) * 2] = m_run[hb];
        a.ws_ml[(slot * a.H + h) * 2 + 1] = l_run[hb];
      }
    }
  }
}

// Merge of the split partials of one (sequence, head): 128 threads x 4 dims.
// Partial s holds o_s / l_s (bf16) with its max m_s and sum l_s (log2 units).
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
    const u32x2_t v = *reinterpret_cast<const u32x2_t*>(a.ws_o + ((s0 + s) * a.H + h) * kDV + d);
    const float w = l > 0.f ? fast_exp2(ml[0] - M) * l : 0.f;
    den += w;
    const float x[4] = {__uint_as_float(v[0] << 16), __uint_as_float(v[0] & 0xFFFF0000u),
                        __uint_as_float(v[1] << 16), __uint_as_float(v[1] & 0xFFFF0000u)};
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] = l > 0.f ? fmaf(w, x[e], acc[e]) : acc[e];
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
  // bf16 partial outputs, then (max, sum) pairs, in floats
  return static_cast<size_t>(a.n_seqs) * a.n_splits * a.H * (kDV / 2 + 2);
}

void launch_mla(const MlaArgs& a0, hipStream_t st) {
  MlaArgs a = a0;
  if (a.n_splits > 1)
    a.ws_ml = reinterpret_cast<float*>(a.ws_o + static_cast<size_t>(a.n_seqs) * a.n_splits * a.H * kDV);
  const int hb = a.H > 64 ? 2 : 1;
  const dim3 grid(a.n_splits, a.n_seqs, (a.H + 64 * hb - 1) / (64 * hb));
  const TimedLaunch tl = timing_prepare(kTimeMla);
  if (hb == 2)
    hipExtLaunchKernelGGL(mla_kernel<2>, grid, dim3(256), 0, st, tl.start, tl.stop, 0, a);
  else
    hipExtLaunchKernelGGL(mla_kernel<1>, grid, dim3(256), 0, st, tl.start, tl.stop, 0, a);
  VKV_HIP(hipGetLastError());
  timing_commit(tl);
  if (a.n_splits > 1) {
    hipLaunchKernelGGL(mla_combine_kernel, dim3(a.H, a.n_seqs), dim3(128), 0, st, a);
    VKV_HIP(hipGetLastError());
  }
}

}  // namespace vkv
