// vkv_decode.hip -- decode attention over paged affine (4/8-bit) bf16 KV on
// gfx950 matrix cores.
//
// Semantics: quantizedScaledDotProductAttention
// (Libraries/MLXLMCommon/KVCache.swift:1909-1997) for one query token per
// sequence: queries scaled in bf16, scores q.dequant(K), softmax, P.dequant(V),
// fp32 accumulation, output rounded to bf16.  Split-K partials are merged as
// sdpa_vector_2pass_2 merges them
// (Source/Cmlx/mlx-generated/metal/sdpa_vector.h:320-394).
//
// Why matrix cores: with 4 query heads per KV head every 4-bit KV byte feeds
// about 7 multiply-adds; at 8 TB/s that is ~110 TFLOP/s of fp32 FMA, more
// than the vector ALUs sustain.  Both contractions therefore run as
// 16x16x32 bf16 MFMAs directly on the codes:
//   * a 4-bit code c enters as bf16(128 + c), bit pattern 0x4300 | c, which
//     is exact; an 8-bit code is split into nibbles c = 16*hi + lo, the hi
//     half meeting a partner operand pre-scaled by 16 (exact in bf16);
//   * per-(token, group) scale s and bias b are applied around the
//     contraction:  q.(s*c + b) = s * q.(128 + c) + (b - 128 s) * sum(q), and
//     sum_t p_t (s_t c_t + b_t) = sum_t P_t (128 + c_t)
//                                 + sum_t p_t b_t - 128 * sum_t P_t
//     with P_t = p_t s_t carried as two bf16 operands (hi + lo, about 16
//     significant bits): a single bf16 P would put a 2^-9 relative error on
//     the code part s*c, which the bias then cancels only partly.  The
//     offset sum uses the same hi + lo values the MFMA consumed, so it
//     cancels to fp32 rounding.  (For 8-bit the offset is 128 + 16*128.)
//
// Work decomposition: a workgroup (4 waves) owns one (partition of 32-token
// blocks, kv head, sequence) and its waves take the partition's blocks round
// robin.  Lane = 16*lg + lrow.  The score MFMA (A = queries, B = key codes)
// leaves token lrow of the tile and query head 4*lg + i in accumulator
// register i; the output MFMA (A = value codes, B = probabilities) leaves
// value dim 16*tile + 4*lg + i and query head lrow.  Probabilities move
// between the two layouts through a per-wave LDS tile.  The running max is
// refreshed lazily (only when a block's max exceeds it by more than kTau),
// which keeps the accumulator rescale off the common path; probabilities are
// then bounded by e^kTau, well inside bf16 range.
#include "vkv_device.h"
#include "vkv_internal.h"

namespace vkv {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr float kTau = 8.0f;
constexpr int kWaves = 4;

__device__ __forceinline__ f32x4_t mfma(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// 8 nibbles -> 8 bf16 (128 + nibble); register p holds nibbles (p, p + 4).
__device__ __forceinline__ u32x4_t nib_magic(uint32_t w) {
  u32x4_t r;
  r[0] = (w & 0x000F000Fu) | 0x43004300u;
  r[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  r[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  r[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return r;
}

// 8 bytes (x then y) -> low / high nibbles as bf16 (128 + nibble); register
// order (b0, b2), (b1, b3) of x, then of y.
__device__ __forceinline__ void byte_magic(uint32_t x, uint32_t y, u32x4_t& lo, u32x4_t& hi) {
  lo[0] = (x & 0x000F000Fu) | 0x43004300u;
  lo[1] = ((x >> 8) & 0x000F000Fu) | 0x43004300u;
  lo[2] = (y & 0x000F000Fu) | 0x43004300u;
  lo[3] = ((y >> 8) & 0x000F000Fu) | 0x43004300u;
  hi[0] = ((x >> 4) & 0x000F000Fu) | 0x43004300u;
  hi[1] = ((x >> 12) & 0x000F000Fu) | 0x43004300u;
  hi[2] = ((y >> 4) & 0x000F000Fu) | 0x43004300u;
  hi[3] = ((y >> 12) & 0x000F000Fu) | 0x43004300u;
}

// Dim (within an 8-dim unit) / token (within an 8-token group) carried by
// MFMA K element j of a lane: 4-bit pairs (p, p+4), 8-bit pairs (0,2),(1,3).
template <int BITS>
__device__ __forceinline__ int kslot(int j) {
  if constexpr (BITS == 4) return (j & 1) ? (j >> 1) + 4 : (j >> 1);
  const int r = j & 3;
  return (j & 4) | (r == 1 ? 2 : r == 2 ? 1 : r);
}
// inverse of kslot (both maps are involutions for 8-bit)
template <int BITS>
__device__ __forceinline__ int kpos(int q) {
  if constexpr (BITS == 4) return q < 4 ? 2 * q : 2 * (q - 4) + 1;
  return kslot<8>(q);
}

template <int N>
__device__ __forceinline__ float ror(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + N, 0xF, 0xF, false));
}
// reductions over the 16 lanes of a DPP row
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, ror<8>(x));
  x = fmaxf(x, ror<4>(x));
  x = fmaxf(x, ror<2>(x));
  return fmaxf(x, ror<1>(x));
}
__device__ __forceinline__ float row16_sum(float x) {
  x += ror<8>(x);
  x += ror<4>(x);
  x += ror<2>(x);
  return x + ror<1>(x);
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// N consecutive words with the widest loads the count allows (the address
// is aligned to the load width by the chunk format).
template <int N>
__device__ __forceinline__ void load_words(const uint8_t* p, uint32_t* out) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int v = 0; v < N / 4; v++) {
      const u32x4_t x = reinterpret_cast<const u32x4_t*>(p)[v];
#pragma unroll
      for (int e = 0; e < 4; e++) out[4 * v + e] = x[e];
    }
  } else if constexpr (N % 2 == 0) {
#pragma unroll
    for (int v = 0; v < N / 2; v++) {
      const u32x2_t x = reinterpret_cast<const u32x2_t*>(p)[v];
      out[2 * v] = x[0];
      out[2 * v + 1] = x[1];
    }
  } else {
#pragma unroll
    for (int v = 0; v < N; v++) out[v] = reinterpret_cast<const uint32_t*>(p)[v];
  }
}

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

template <int BITS, int D>
__global__ void __launch_bounds__(256, 2) qdecode_mfma_kernel(DecodeArgs a) {
  constexpr int G = D / 64;                          // quantization groups per row
  constexpr int KS = D / 32;                         // 32-dim K steps
  constexpr int NT = D / 16;                         // 16-dim output tiles
  constexpr int KW = (BITS == 4) ? KS : 2 * KS;      // key words per lane per token
  constexpr int VW = (BITS == 4) ? NT : 2 * NT;      // value words per lane
  constexpr int ROW = D * BITS / 8;                  // key code bytes per token
  constexpr int SBV = 4 * G;                         // scale/bias values per token
  constexpr int NP = (BITS == 4) ? 1 : 2;            // probability tiles (x1, x16)
  constexpr float MAG = (BITS == 4) ? 128.0f : 2176.0f;
  constexpr float C0 = (BITS == 4) ? 8.0f : 128.0f;  // code midpoint

  // One LDS region serves three phases: the queries (qf) until the MFMA
  // operands are built, the per-wave probability tiles (ptile: x1 / x16
  // copies, each split into bf16 hi + lo parts) during the block loop, and
  // the per-wave output staging (fin_o) after it.
  constexpr int QF_BYTES = 16 * D * 4;
  constexpr int PT_BYTES = kWaves * NP * 2 * G * 16 * 32 * 2;
  constexpr int FIN_BYTES = kWaves * 16 * (D + 1) * 4;
  constexpr int U1 = QF_BYTES > PT_BYTES ? QF_BYTES : PT_BYTES;
  __shared__ __attribute__((aligned(16))) uint8_t smem_u[U1 > FIN_BYTES ? U1 : FIN_BYTES];
  float(*qf)[D] = reinterpret_cast<float(*)[D]>(smem_u);
  float(*fin_o)[16][D + 1] = reinterpret_cast<float(*)[16][D + 1]>(smem_u);
  typedef uint16_t ptile_t[NP][2][G][16][32];
  ptile_t* ptile = reinterpret_cast<ptile_t*>(smem_u);
  __shared__ float sqs[16][G];
  __shared__ float fin_s[kWaves][16][2 + G];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, lrow = lane & 15, lg = lane >> 4;
  const int part = blockIdx.x, hk = blockIdx.y, seq = blockIdx.z;
  const int rep = a.rep;
  const int len = a.seq_lens ? a.seq_lens[seq] : a.max_len;
  const int nblk = (len + 31) >> 5;
  const int b0 = part * a.part_blocks;
  const int b1 = min(nblk, b0 + a.part_blocks);

  // ---- queries of this kv head's query heads, scaled in bf16
  const float scale_t = round_to<kBF16>(a.scale);
  for (int i = tid; i < 16 * D; i += 256) {
    const int r = i / D, d = i % D;
    float v = 0.0f;
    if (r < rep) {
      const int64_t h = static_cast<int64_t>(hk) * rep + r;
      v = round_to<kBF16>(bf16_to_f32(a.q[seq * a.q_ss + h * a.q_sh + d]) * scale_t);
    }
    qf[r][d] = v;
  }
  __syncthreads();
  if (tid < 16 * G) {
    const int r = tid / G, g = tid % G;
    float s = 0.0f;
    for (int d = 0; d < 64; d++) s += qf[r][g * 64 + d];
    sqs[r][g] = s;
  }
  // score-MFMA A operands: row = head lrow, K = the 8 dims of unit 4s + lg
  u32x4_t aq[KS];
  u32x4_t aq16[BITS == 8 ? KS : 1];
#pragma unroll
  for (int s = 0; s < KS; s++) {
    const int unit = 4 * s + lg;
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const float x0 = qf[lrow][8 * unit + kslot<BITS>(2 * p)];
      const float x1 = qf[lrow][8 * unit + kslot<BITS>(2 * p + 1)];
      aq[s][p] = pack_bf16(x0, x1);
      if constexpr (BITS == 8) aq16[s][p] = pack_bf16(16.0f * x0, 16.0f * x1);
    }
  }
  __syncthreads();
  float sq[4][G];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int g = 0; g < G; g++) sq[i][g] = sqs[4 * lg + i][g];

  f32x4_t oacc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) oacc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run[4], l_run[4], corr[4][G];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.0f;
#pragma unroll
    for (int g = 0; g < G; g++) corr[i][g] = 0.0f;
  }

  const int subs = a.block_size >> 5;  // 32-token sub-blocks per pool block
  for (int b = b0 + wave; b < b1; b += kWaves) {
    const int64_t blk = a.table[static_cast<int64_t>(seq) * a.table_stride + b / subs];
    const int sub = b % subs;
    const uint8_t* chunk = a.base + blk * a.block_bytes + static_cast<int64_t>(hk) * a.head_bytes;
    // ---- loads: key codes and scale/bias of tokens lrow, lrow+16; value codes
    uint32_t kw[2][KW];
    uint32_t sb[2][SBV / 2];
#pragma unroll
    for (int tile = 0; tile < 2; tile++) {
      const int t = sub * 32 + tile * 16 + lrow;
      load_words<KW>(chunk + a.kc_off + t * ROW + lg * KW * 4, kw[tile]);
      load_words<SBV / 2>(chunk + a.sb_off + t * SBV * 2, sb[tile]);
    }
    uint32_t vw[VW];
    load_words<VW>(chunk + a.vc_off + sub * 32 * ROW + (lg * 16 + lrow) * VW * 4, vw);

    // ---- scores of query heads 4*lg + i for tokens (tile*16 + lrow)
    float sc[2][4];
#pragma unroll
    for (int tile = 0; tile < 2; tile++) {
      f32x4_t acc[G];
#pragma unroll
      for (int g = 0; g < G; g++) {
        acc[g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k2 = 0; k2 < 2; k2++) {
          const int s = 2 * g + k2;
          if constexpr (BITS == 4) {
            acc[g] = mfma(aq[s], nib_magic(kw[tile][s]), acc[g]);
          } else {
            u32x4_t lo, hi;
            byte_magic(kw[tile][2 * s], kw[tile][2 * s + 1], lo, hi);
            acc[g] = mfma(aq16[s], hi, acc[g]);
            acc[g] = mfma(aq[s], lo, acc[g]);
          }
        }
      }
      const int tok = b * 32 + tile * 16 + lrow;
      float ks[G], u[G];
#pragma unroll
      for (int g = 0; g < G; g++) {
        const uint32_t w = sb[tile][g];  // (scale, bias) of key group g
        ks[g] = bf_lo(w);
        u[g] = fmaf(-MAG, ks[g], bf_hi(w));
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float s = 0.0f;
#pragma unroll
        for (int g = 0; g < G; g++) s = fmaf(u[g], sq[i][g], s);
#pragma unroll
        for (int g = 0; g < G; g++) s = fmaf(ks[g], acc[g][i], s);
        sc[tile][i] = (tok < len && 4 * lg + i < rep) ? s : -INFINITY;
      }
    }

    // ---- online softmax, max refreshed lazily
    float mx[4];
    bool need = false;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      mx[i] = row16_max(fmaxf(sc[0][i], sc[1][i]));
      need |= mx[i] > m_run[i] + kTau;
    }
    if (__any(need)) {
      float alpha[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const bool up = mx[i] > m_run[i] + kTau;
        alpha[i] = up ? (m_run[i] == -INFINITY ? 0.0f : __expf(m_run[i] - mx[i])) : 1.0f;
        if (up) m_run[i] = mx[i];
        l_run[i] *= alpha[i];
#pragma unroll
        for (int g = 0; g < G; g++) corr[i][g] *= alpha[i];
      }
      // output accumulators carry head lrow: alpha of head lrow lives in
      // register (lrow % 4) of lane group lrow / 4
      float al = 1.0f;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float v = __shfl(alpha[i], 16 * (lrow >> 2));
        if ((lrow & 3) == i) al = v;
      }
#pragma unroll
      for (int t = 0; t < NT; t++) oacc[t] *= al;
    }
    float p[2][4];
#pragma unroll
    for (int tile = 0; tile < 2; tile++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        p[tile][i] = sc[tile][i] == -INFINITY ? 0.0f : __expf(sc[tile][i] - m_run[i]);
        l_run[i] += p[tile][i];
      }

    // ---- probability operands p*s_v (bf16) into LDS in the value operand's
    // K order; the same rounded values feed the offset correction.  The
    // correction re-centres the codes on their midpoint C0: with
    // P = bf16(p s) = p s (1 + e), the MFMA term sum P (MAG + c) plus
    // sum p (b + C0 s) - (MAG + C0) sum P equals the exact result up to
    // sum p s (c - C0) e, an error of the size of bf16-rounding the value
    // itself rather than its (often much larger) code part s*c.
    const int col0 = kpos<BITS>(lrow & 7) + (lrow & 8);
    const int col1 = col0 + 16;
#pragma unroll
    for (int g = 0; g < G; g++) {
      const uint32_t v0 = sb[0][G + g], v1 = sb[1][G + g];  // (scale, bias) of value group g
      const float vs0 = bf_lo(v0), vs1 = bf_lo(v1);
      const float vb0 = fmaf(C0, vs0, bf_hi(v0)), vb1 = fmaf(C0, vs1, bf_hi(v1));
#pragma unroll
      for (int i = 0; i < 4; i++) {
        // p*s as hi + lo bf16 (about 16 significant bits between them)
        const float pv0 = p[0][i] * vs0, pv1 = p[1][i] * vs1;
        const uint32_t ph = pack_bf16(pv0, pv1);
        const uint32_t pl = pack_bf16(pv0 - bf_lo(ph), pv1 - bf_hi(ph));
        uint16_t* rh = ptile[wave][0][0][g][4 * lg + i];
        uint16_t* rl = ptile[wave][0][1][g][4 * lg + i];
        rh[col0] = static_cast<uint16_t>(ph);
        rh[col1] = static_cast<uint16_t>(ph >> 16);
        rl[col0] = static_cast<uint16_t>(pl);
        rl[col1] = static_cast<uint16_t>(pl >> 16);
        if constexpr (BITS == 8) {  // x16 copies are exact rescalings
          const uint32_t ph16 = pack_bf16(16.0f * bf_lo(ph), 16.0f * bf_hi(ph));
          const uint32_t pl16 = pack_bf16(16.0f * bf_lo(pl), 16.0f * bf_hi(pl));
          uint16_t* rh16 = ptile[wave][1][0][g][4 * lg + i];
          uint16_t* rl16 = ptile[wave][1][1][g][4 * lg + i];
          rh16[col0] = static_cast<uint16_t>(ph16);
          rh16[col1] = static_cast<uint16_t>(ph16 >> 16);
          rl16[col0] = static_cast<uint16_t>(pl16);
          rl16[col1] = static_cast<uint16_t>(pl16 >> 16);
        }
        float c = fmaf(p[0][i], vb0, corr[i][g]);
        c = fmaf(p[1][i], vb1, c);
        c = fmaf(-(MAG + C0), bf_lo(ph) + bf_lo(pl), c);
        corr[i][g] = fmaf(-(MAG + C0), bf_hi(ph) + bf_hi(pl), c);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- O^T[dim][head] += V^T . P'^T
    u32x4_t bp[NP][2][G];
#pragma unroll
    for (int n = 0; n < NP; n++)
#pragma unroll
      for (int hl = 0; hl < 2; hl++)
#pragma unroll
        for (int g = 0; g < G; g++)
          bp[n][hl][g] = *reinterpret_cast<const u32x4_t*>(&ptile[wave][n][hl][g][lrow][8 * lg]);
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const int g = t / 4;
      if constexpr (BITS == 4) {
        const u32x4_t av = nib_magic(vw[t]);
        oacc[t] = mfma(av, bp[0][0][g], oacc[t]);
        oacc[t] = mfma(av, bp[0][1][g], oacc[t]);
      } else {
        u32x4_t lo, hi;
        byte_magic(vw[2 * t], vw[2 * t + 1], lo, hi);
        oacc[t] = mfma(hi, bp[1][0][g], oacc[t]);
        oacc[t] = mfma(hi, bp[1][1][g], oacc[t]);
        oacc[t] = mfma(lo, bp[0][0][g], oacc[t]);
        oacc[t] = mfma(lo, bp[0][1][g], oacc[t]);
      }
    }
    // the next block rewrites this wave's tile only after every lane read it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- per-wave results: m, l, corrections (per head, token-lane layout)
  float lsum[4], csum[4][G];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    lsum[i] = row16_sum(l_run[i]);
#pragma unroll
    for (int g = 0; g < G; g++) csum[i][g] = row16_sum(corr[i][g]);
  }
  if (lrow == 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      fin_s[wave][4 * lg + i][0] = m_run[i];
      fin_s[wave][4 * lg + i][1] = lsum[i];
#pragma unroll
      for (int g = 0; g < G; g++) fin_s[wave][4 * lg + i][2 + g] = csum[i][g];
    }
  }
  __syncthreads();
  // output tile t, register i: value dim 16t + 4lg + i, head lrow
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const float c = fin_s[wave][lrow][2 + t / 4];
#pragma unroll
    for (int i = 0; i < 4; i++) fin_o[wave][lrow][16 * t + 4 * lg + i] = oacc[t][i] + c;
  }
  __syncthreads();

  // ---- merge the 4 waves, then write the partition's partial or the output
  for (int idx = tid; idx < rep * D; idx += 256) {
    const int r = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; w++) M = fmaxf(M, fin_s[w][r][0]);
    float o = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
      const float mw = fin_s[w][r][0];
      if (mw == -INFINITY) continue;
      const float f = __expf(mw - M);
      o = fmaf(f, fin_o[w][r][d], o);
      L = fmaf(f, fin_s[w][r][1], L);
    }
    const int64_t h = static_cast<int64_t>(hk) * rep + r;
    if (a.n_parts == 1) {
      a.out[seq * a.o_ss + h * a.o_sh + d] = f32_to_bf16(L > 0.0f ? o / L : 0.0f);
    } else {
      const int64_t base = (static_cast<int64_t>(seq) * a.Hq + h) * a.n_parts + part;
      a.ws_o[base * D + d] = o;
      if (d == 0) {
        a.ws_ml[base * 2] = M == -INFINITY ? -3.402823466e38f : M;
        a.ws_ml[base * 2 + 1] = L;
      }
    }
  }
}

// Merge of the partition partials (sdpa_vector.h:320-394).
__global__ void __launch_bounds__(256) qdecode_combine_kernel(DecodeArgs a, int D) {
  const int64_t rh = blockIdx.x;  // seq * Hq + h
  const int64_t seq = rh / a.Hq;
  const int64_t h = rh % a.Hq;
  const float* ml = a.ws_ml + rh * a.n_parts * 2;
  float M = -3.402823466e38f;
  for (int p = 0; p < a.n_parts; p++) M = fmaxf(M, ml[2 * p]);
  float L = 0.0f;
  for (int p = 0; p < a.n_parts; p++) L += __expf(ml[2 * p] - M) * ml[2 * p + 1];
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float o = 0.0f;
    for (int p = 0; p < a.n_parts; p++) o += __expf(ml[2 * p] - M) * a.ws_o[(rh * a.n_parts + p) * D + d];
    a.out[seq * a.o_ss + h * a.o_sh + d] = f32_to_bf16(L > 0.0f ? o / L : 0.0f);
  }
}

bool qdecode_supported(int dtype, int bits, int D, int block_size, int rep, int group) {
  return dtype == kBF16 && (bits == 4 || bits == 8) && (D == 64 || D == 128) &&
         block_size % 32 == 0 && rep >= 1 && rep <= 16 && group == 64;
}

void launch_qdecode(const DecodeArgs& a, int bits, int D, int n_seqs, hipStream_t st) {
  dim3 grid(a.n_parts, a.Hkv, n_seqs);
#define VKV_QD(B, DD) hipLaunchKernelGGL((qdecode_mfma_kernel<B, DD>), grid, dim3(256), 0, st, a)
  if (bits == 4) {
    if (D == 64) VKV_QD(4, 64);
    else VKV_QD(4, 128);
  } else {
    if (D == 64) VKV_QD(8, 64);
    else VKV_QD(8, 128);
  }
#undef VKV_QD
  VKV_HIP(hipGetLastError());
  if (a.n_parts > 1) {
    hipLaunchKernelGGL(qdecode_combine_kernel, dim3(static_cast<unsigned>(n_seqs) * a.Hq), dim3(128), 0,
                       st, a, D);
    VKV_HIP(hipGetLastError());
  }
}

}  // namespace vkv
