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
// Arithmetic.  Both contractions run as 16x16x32 bf16 MFMAs directly on the
// codes, so the vector ALUs only unpack codes and run the softmax:
//   * a 4-bit code c enters as bf16(128 + c), bit pattern 0x4300 | c, which
//     is exact; an 8-bit code c = 16*hi + lo enters as two operands,
//     bf16(128 + lo) = 0x4300 | lo and bf16(2048 + 16*hi) = 0x4500 | hi, whose
//     sum is c + 2176 (MAG);
//   * per-(token, group) scale s and bias b are applied around the
//     contraction:  q.(s*c + b) = s * q.(MAG + c) + (b - MAG s) * sum(q), and
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
// Workgroup = 4 waves = (partition of steps, kv head and head group,
// sequence); waves take
// the partition's steps round robin, with the next step's loads in flight
// while the current one computes when the per-step operands fit in
// registers twice.  A sequence that fits one partition is written directly;
// longer ones leave per-partition partials that qdecode_combine_kernel
// merges.  (Merging in the last workgroup to finish would need device-scope
// release/acquire fences, which on gfx950 write back and invalidate the
// XCD's whole L2 and cost more than the extra launch.)
#include <utility>

#include "vkv_device.h"
#include "vkv_internal.h"

namespace vkv {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
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
constexpr int kWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxPartSteps = 64;  // 64-token steps per workgroup partition, at most

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

// The bf16 exponent patterns OR-ed onto the codes, held in VGPRs the
// compiler cannot see through: with both the mask and the pattern as
// literals it emits v_and + v_or, with the pattern in a register one
// v_and_or_b32.
struct Magic {
  uint32_t m128, m2048;  // 0x43004300 (128 + c), 0x45004500 (2048 + 16 c)
  __device__ __forceinline__ Magic() : m128(0x43004300u), m2048(0x45004500u) {
    asm volatile("" : "+v"(m128), "+v"(m2048));
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
    return __builtin_amdgcn_update_dpp(0u, x, 0x120 + (16 - K), 0xF, 0xF, false);
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

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// LDS-only barrier: orders LDS traffic across the workgroup but leaves
// global loads in flight (a plain __syncthreads waits for them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int BITS, int D, int HP>
struct QD {
  static constexpr int G = D / 64;            // quantization groups per row
  static constexpr int PP = 16 / HP;          // token parts of a score tile
  static constexpr int TT = 4 / PP;           // score tiles per 64-token step
  static constexpr int SPW = 4 / PP;          // lane groups per part
  static constexpr int SL = D * PP / 32;      // score K slices (8 dims per lane)
  static constexpr int UW = BITS / 4;         // words per 8-dim unit
  static constexpr int RUN = (D / 32) * UW;   // key words of one lane-group run
  static constexpr int NT = D / 16;           // 16-dim output tiles
  static constexpr int VW = NT * UW;          // value words per lane per sub-block
  static constexpr int ROW = D * BITS / 8;    // key code bytes per token
  static constexpr int SBW = 2 * G;           // scale/bias words per token (K, V)
  static constexpr int QROW = 16 * SPW + 1;   // query-table entries per slice
  static constexpr float MAG = (BITS == 4) ? 128.0f : 2176.0f;
  static constexpr float C0 = (BITS == 4) ? 8.0f : 128.0f;
  // per-step operand registers; steps are double buffered when they fit
  static constexpr int BUF = D * UW / 4 + HP * D / 32;
  static constexpr bool kPrefetch = BUF <= 48;

  struct Buf {
    uint32_t kw[TT][PP][RUN];    // key words of this lane's token, per tile
    uint32_t sb[TT][4][SBW];     // scale/bias of the 4 scored tokens, per tile
    uint32_t vw[2][VW];          // value words, per 32-token sub-block
  };
};

template <int BITS, int D, int HP>
__global__ void __launch_bounds__(256, (D >= 256) ? 1 : 2) qdecode_kernel(DecodeArgs a) {
  using C = QD<BITS, D, HP>;
  constexpr int G = C::G, PP = C::PP, TT = C::TT, SPW = C::SPW, SL = C::SL;
  constexpr int RUN = C::RUN, NT = C::NT, VW = C::VW, ROW = C::ROW, SBW = C::SBW;
  constexpr int QROW = C::QROW;
  constexpr float MAG = C::MAG, C0 = C::C0;
  using Buf = typename C::Buf;

  // LDS: the query table (score B operands) during the step loop, the
  // per-wave results after it.
  constexpr int QT_BYTES = SL * QROW * 16;
  constexpr int FIN_BYTES = kWaves * HP * D * 4;
  __shared__ __attribute__((aligned(16))) uint8_t smem[QT_BYTES > FIN_BYTES ? QT_BYTES : FIN_BYTES];
  __shared__ float qf[HP][D + 1];
  __shared__ float sqs[HP][G];
  __shared__ int32_t sblk[2 * kMaxPartSteps];  // pool block of each sub-block
  __shared__ float fin_s[kWaves][HP][2];
  u32x4_t* qtab = reinterpret_cast<u32x4_t*>(smem);
  float(*fin_o)[HP][D] = reinterpret_cast<float(*)[HP][D]>(smem);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int lane = tid & 63, n = lane & 15, lg = lane >> 4;
  const int part = blockIdx.x, seq = blockIdx.z;
  const int rep = a.rep;
  const int n_hg = (rep + HP - 1) / HP;  // head groups of HP query heads
  const int hk = blockIdx.y / n_hg, hg = blockIdx.y % n_hg;
  const int nh = min(HP, rep - hg * HP);  // query heads of this workgroup
  // first query head of the group, and its (sequence, head) row
  const int64_t hq0 = static_cast<int64_t>(hk) * rep + hg * HP;
  const int64_t rh0 = static_cast<int64_t>(seq) * a.Hq + hq0;
  const int len = a.seq_lens ? a.seq_lens[seq] : a.max_len;
  const int nstep = (len + 63) >> 6;
  // balanced partitions: parts_used pieces of at most part_steps steps
  const int parts_used = (nstep + a.part_steps - 1) / a.part_steps;
  if (part >= parts_used) {
    if (nstep == 0 && part == 0) {  // empty sequence: zero output
      for (int idx = tid; idx < nh * D; idx += 256)
        a.out[seq * a.o_ss + (hq0 + idx / D) * a.o_sh + idx % D] = 0;
    }
    return;
  }
  const int span = (nstep + parts_used - 1) / parts_used;  // <= part_steps
  const int st0 = part * span;                              // < nstep
  const int st1 = min(nstep, st0 + span);
  const int nsub = (len + 31) >> 5;
  const int subs = a.block_size >> 5;  // 32-token sub-blocks per pool block
  const int32_t* table = a.table + static_cast<int64_t>(seq) * a.table_stride;
  const uint8_t* head_base = a.base + static_cast<int64_t>(hk) * a.head_bytes;

  // this lane's roles: score column (part p, head h); key-operand lane
  // group (part pA, unit slot wA)
  const int p = n / HP, h = n % HP;
  const int pA = lg / SPW, wA = lg % SPW;

  // direct: read the block table from memory (the first step, issued
  // before the LDS copy of the partition's table slice exists)
  auto load_step = [&](int stp, Buf& b, bool direct) {
    const uint8_t* cb[2];
    int t0[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const int sbi = min(2 * stp + s, nsub - 1);
      const int64_t blk =
          direct ? table[sbi / subs] : __builtin_amdgcn_readfirstlane(sblk[sbi - 2 * st0]);
      cb[s] = head_base + blk * a.block_bytes;
      t0[s] = (sbi % subs) * 32;
    }
#pragma unroll
    for (int tau = 0; tau < TT; tau++) {
      {  // key row of token 8 (n / 4) + off(q, n % 4) of part (tau, pA)
        const int c = tau * PP + pA, s = c >> 1, q = c & 1;
        const int t = t0[s] + 8 * (n >> 2) + tok_off<BITS>(q, n & 3);
        const uint8_t* row = cb[s] + a.kc_off + static_cast<int64_t>(t) * ROW;
#pragma unroll
        for (int rho = 0; rho < PP; rho++)
          load_words<RUN>(row + (rho * SPW + wA) * RUN * 4, b.kw[tau][rho]);
      }
      {  // scale/bias of the tokens this lane scores (column part p)
        const int c = tau * PP + p, s = c >> 1, q = c & 1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int t = t0[s] + 8 * lg + tok_off<BITS>(q, i);
          load_words<SBW>(cb[s] + a.sb_off + static_cast<int64_t>(t) * SBW * 4, b.sb[tau][i]);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < 2; s++)
      load_words<VW>(cb[s] + a.vc_off + t0[s] * ROW + (lg * 16 + n) * VW * 4, b.vw[s]);
  };

  // Global loads complete in issue order (one wait counter), so the set-up
  // reads (table slice, queries) are issued before the first step's KV
  // loads, which then stay in flight while the set-up uses them.  Every
  // load here is unconditional (clamped indices): a load under a branch
  // makes the compiler wait for all outstanding loads at the join.
  constexpr int QPT = (HP * D + 255) / 256;  // query elements per thread
  const int n_sub_part = 2 * (st1 - st0);  // <= 2 * kMaxPartSteps <= 256
  const int32_t my_blk = table[min(2 * st0 + tid, nsub - 1) / subs];
  uint16_t qraw[QPT];
#pragma unroll
  for (int j = 0; j < QPT; j++) {
    const int i = tid + 256 * j, r = min(i / D, nh - 1), d = i % D;
    qraw[j] = a.q[seq * a.q_ss + (hq0 + r) * a.q_sh + d];
  }
  Buf bufA, bufB;
  int step = st0 + wave;
  load_step(min(step, st1 - 1), bufA, true);  // in flight during the set-up
  const Magic mg;
  if (tid < n_sub_part) sblk[tid] = my_blk;  // the partition's block-table slice
  // ---- queries of the group's heads, scaled in bf16; rows >= nh are 0
  const float scale_t = round_to<kBF16>(a.scale);
#pragma unroll
  for (int j = 0; j < QPT; j++) {
    const int i = tid + 256 * j;
    const float v = round_to<kBF16>(bf16_to_f32(qraw[j]) * scale_t);
    if (i < HP * D) qf[i / D][i % D] = (i / D < nh) ? v : 0.0f;
  }
  lds_barrier();
  // query table: entry (slice sg, column nn, unit slot w) holds the 8 dims
  // of unit sg * SPW + w of head nn % HP in the key operand's K order;
  // entry 16 * SPW of every slice is zero (lanes outside the column's part)
  for (int e = tid; e < SL * QROW; e += 256) {
    const int sg = e / QROW, r = e % QROW;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (r < 16 * SPW) {
      const int nn = r / SPW, w = r % SPW;
      const int unit = sg * SPW + w;
      const float* qrow = qf[nn % HP];
#pragma unroll
      for (int pr = 0; pr < 4; pr++)
        v[pr] = pack_bf16(qrow[8 * unit + kslot<BITS>(2 * pr)], qrow[8 * unit + kslot<BITS>(2 * pr + 1)]);
    }
    qtab[e] = v;
  }
  // sum of each head's bf16 queries per group: 32 lanes per (head, group)
  for (int rg = tid >> 5; rg < HP * G; rg += 8) {
    const int r = rg / G, g = rg % G, j = tid & 31;
    float s = qf[r][g * 64 + j] + qf[r][g * 64 + j + 32];
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) s += __shfl_xor(s, o, 32);
    if (j == 0) sqs[r][g] = s;
  }
  lds_barrier();
  float sq[G];
#pragma unroll
  for (int g = 0; g < G; g++) sq[g] = sqs[h][g];
  const u32x4_t* qlane = qtab + ((pA == p) ? n * SPW + wA : 16 * SPW);

  f32x4_t oacc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) oacc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f, corr[G];
#pragma unroll
  for (int g = 0; g < G; g++) corr[g] = 0.0f;

  auto compute_step = [&](int stp, const Buf& b) {
    // ---- scores: acc[tau][g] = q . (MAG + c) over group g's dims
    f32x4_t acc[TT][G];
#pragma unroll
    for (int tau = 0; tau < TT; tau++)
#pragma unroll
      for (int g = 0; g < G; g++) acc[tau][g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // query slices are read kQA ahead of their MFMAs; the scheduling
    // barrier keeps the compiler from issuing every slice's LDS read up front
    constexpr int kQA = SL < 4 ? SL : 4;
    u32x4_t qring[kQA];
#pragma unroll
    for (int j = 0; j < kQA; j++) qring[j] = qlane[j * QROW];
#pragma unroll
    for (int sg = 0; sg < SL; sg++) {
      const u32x4_t qb = qring[sg % kQA];
      if (sg + kQA < SL) qring[sg % kQA] = qlane[(sg + kQA) * QROW];
      const int g = sg / (SL / G), rho = sg % PP, k = sg / PP;
#pragma unroll
      for (int tau = 0; tau < TT; tau++) {
        if constexpr (BITS == 4) {
          acc[tau][g] = mfma(nib_magic(b.kw[tau][rho][k], mg), qb, acc[tau][g]);
        } else {
          u32x4_t lo, hi;
          byte_magic(b.kw[tau][rho][2 * k], b.kw[tau][rho][2 * k + 1], mg, lo, hi);
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
          const uint32_t kwd = b.sb[tau][i][g], vwd = b.sb[tau][i][G + g];
          const float ks = bf_lo(kwd);
          s = fmaf(fmaf(-MAG, ks, bf_hi(kwd)), sq[g], s);
          s = fmaf(ks, acc[tau][g][i], s);
          vs[tau][i][g] = bf_lo(vwd);
          vb[tau][i][g] = bf_hi(vwd);
        }
        sc[tau][i] = s;
      }
    if (stp * 64 + 64 > len) {  // the sequence ends inside this step
#pragma unroll
      for (int tau = 0; tau < TT; tau++) {
        const int c = tau * PP + p, s = c >> 1, q = c & 1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const bool ok = stp * 64 + 32 * s + 8 * lg + tok_off<BITS>(q, i) < len;
          sc[tau][i] = ok ? sc[tau][i] : -INFINITY;
#pragma unroll
          for (int g = 0; g < G; g++) {
            vs[tau][i][g] = ok ? vs[tau][i][g] : 0.0f;
            vb[tau][i][g] = ok ? vb[tau][i][g] : 0.0f;
          }
        }
      }
    }

    // ---- online softmax with a lazily refreshed max
    bool need = false;
#pragma unroll
    for (int tau = 0; tau < TT; tau++)
#pragma unroll
      for (int i = 0; i < 4; i++) need |= sc[tau][i] > m_run + kTau;
    if (__builtin_amdgcn_ballot_w64(need)) {
      float mx = -INFINITY;
#pragma unroll
      for (int tau = 0; tau < TT; tau++)
#pragma unroll
        for (int i = 0; i < 4; i++) mx = fmaxf(mx, sc[tau][i]);
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
      // the P.V accumulators of lane n + 16 lg carry head n = h for n < HP
#pragma unroll
      for (int t = 0; t < NT; t++) oacc[t] *= alpha;
    }
    const float m2 = fmaxf(m_run * kLog2e, -3.402823466e38f);
    float pr[TT][4];
#pragma unroll
    for (int tau = 0; tau < TT; tau++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        pr[tau][i] = exp2f(fmaf(sc[tau][i], kLog2e, -m2));
        l_run += pr[tau][i];
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
          float cc = corr[g];
          cc = fmaf(pr[tau][i0], fmaf(C0, vs[tau][i0][g], vb[tau][i0][g]), cc);
          cc = fmaf(pr[tau][i1], fmaf(C0, vs[tau][i1][g], vb[tau][i1][g]), cc);
          cc = fmaf(-(MAG + C0), (h0 + h1) + (bf_lo(pl) + bf_hi(pl)), cc);
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
          const u32x4_t av = nib_magic(b.vw[s][t], mg);
          oacc[t] = mfma(av, bpv[g][0], oacc[t]);
          oacc[t] = mfma(av, bpv[g][1], oacc[t]);
        } else {
          u32x4_t lo, hi;
          byte_magic(b.vw[s][2 * t], b.vw[s][2 * t + 1], mg, lo, hi);
          oacc[t] = mfma(lo, bpv[g][0], oacc[t]);
          oacc[t] = mfma(lo, bpv[g][1], oacc[t]);
          oacc[t] = mfma(hi, bpv[g][0], oacc[t]);
          oacc[t] = mfma(hi, bpv[g][1], oacc[t]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    });
  };

  if constexpr (C::kPrefetch) {
    // The next step's loads are issued unconditionally (clamped to the last
    // step, whose data is then re-read from cache): a conditional load
    // makes the compiler merge the buffer registers at the join, which
    // waits for the loads right after issuing them.
    while (step < st1) {
      const int nx = step + kWaves;
      load_step(min(nx, st1 - 1), bufB, false);
      __builtin_amdgcn_sched_barrier(0);  // issue the loads before any compute
      compute_step(step, bufA);
      if (nx >= st1) break;
      const int nx2 = nx + kWaves;
      load_step(min(nx2, st1 - 1), bufA, false);
      __builtin_amdgcn_sched_barrier(0);
      compute_step(nx, bufB);
      step = nx2;
    }
  } else {
    while (step < st1) {
      compute_step(step, bufA);
      step += kWaves;
      if (step < st1) load_step(step, bufA, false);
    }
  }

  // ---- per-wave totals of head h: sum over the parts of the row, then rows
  float lsum = l_run, csum[G];
#pragma unroll
  for (int g = 0; g < G; g++) csum[g] = corr[g];
  sfor<PP>([&](auto k_) {
    constexpr int k = decltype(k_)::value;
    if constexpr (k > 0 && (k & (k - 1)) == 0) {  // offsets HP, 2 HP, ... below 16
      lsum += row_readf<k * HP>(lsum);
#pragma unroll
      for (int g = 0; g < G; g++) csum[g] += row_readf<k * HP>(csum[g]);
    }
  });
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
#pragma unroll
  for (int g = 0; g < G; g++) {
    csum[g] += __shfl_xor(csum[g], 16);
    csum[g] += __shfl_xor(csum[g], 32);
  }
  __syncthreads();  // the query table is dead; its LDS becomes fin_o
  if (n < HP && lg == 0) {
    fin_s[wave][n][0] = m_run;
    fin_s[wave][n][1] = lsum;
  }
  if (n < nh) {
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const float cg = csum[t / (NT / G)];
#pragma unroll
      for (int i = 0; i < 4; i++) fin_o[wave][n][16 * t + 4 * lg + i] = oacc[t][i] + cg;
    }
  }
  __syncthreads();

  // ---- merge the waves; write the output or this partition's partial
  for (int idx = tid; idx < nh * D; idx += 256) {
    const int r = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; w++) M = fmaxf(M, fin_s[w][r][0]);
    float o = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
      const float mw = fin_s[w][r][0];
      if (mw == -INFINITY) continue;
      const float f = exp2f((mw - M) * kLog2e);
      o = fmaf(f, fin_o[w][r][d], o);
      L = fmaf(f, fin_s[w][r][1], L);
    }
    if (parts_used == 1) {
      a.out[seq * a.o_ss + (hq0 + r) * a.o_sh + d] = f32_to_bf16(L > 0.0f ? o / L : 0.0f);
    } else {
      const int64_t slot = (rh0 + r) * a.n_parts + part;
      a.ws_o[slot * D + d] = o;
      if (d == 0) {
        a.ws_ml[slot * 2] = M;
        a.ws_ml[slot * 2 + 1] = L;
      }
    }
  }
}

// Merge of the partition partials of sequences longer than one partition
// (sdpa_vector.h:320-394).  Block = one (sequence, query head).
__global__ void __launch_bounds__(256) qdecode_combine_kernel(DecodeArgs a, int D) {
  const int64_t rh = blockIdx.x;  // seq * Hq + h
  const int seq = static_cast<int>(rh / a.Hq);
  const int64_t h = rh % a.Hq;
  const int len = a.seq_lens ? a.seq_lens[seq] : a.max_len;
  const int parts_used = ((len + 63) / 64 + a.part_steps - 1) / a.part_steps;
  if (parts_used <= 1) return;  // written by the partition itself
  const float* ml = a.ws_ml + rh * a.n_parts * 2;
  float M = -INFINITY;
  for (int pp = 0; pp < parts_used; pp++) M = fmaxf(M, ml[2 * pp]);
  float L = 0.0f;
  for (int pp = 0; pp < parts_used; pp++) L = fmaf(exp2f((ml[2 * pp] - M) * kLog2e), ml[2 * pp + 1], L);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    const float* wo = a.ws_o + rh * a.n_parts * D + d;
    float o = 0.0f;
    for (int pp = 0; pp < parts_used; pp++)
      o = fmaf(exp2f((ml[2 * pp] - M) * kLog2e), wo[static_cast<int64_t>(pp) * D], o);
    a.out[seq * a.o_ss + h * a.o_sh + d] = f32_to_bf16(L > 0.0f ? o / L : 0.0f);
  }
}

static int heads_per_part(int rep) { return rep <= 4 ? 4 : 8; }

int qdecode_head_groups(int rep) { return (rep + heads_per_part(rep) - 1) / heads_per_part(rep); }

bool qdecode_supported(int dtype, int bits, int D, int block_size, int rep, int group) {
  return dtype == kBF16 && (bits == 4 || bits == 8) && (D == 64 || D == 128 || D == 256) &&
         block_size % 32 == 0 && rep >= 1 && rep <= 16 && group == 64;
}

template <int BITS, int D>
static void launch_d(const DecodeArgs& a, dim3 grid, hipStream_t st) {
  if (heads_per_part(a.rep) == 4)
    hipLaunchKernelGGL((qdecode_kernel<BITS, D, 4>), grid, dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((qdecode_kernel<BITS, D, 8>), grid, dim3(256), 0, st, a);
}

void launch_qdecode(const DecodeArgs& a, int bits, int D, int n_seqs, hipStream_t st) {
  const dim3 grid(a.n_parts, a.Hkv * qdecode_head_groups(a.rep), n_seqs);
  if (bits == 4) {
    if (D == 64) launch_d<4, 64>(a, grid, st);
    else if (D == 128) launch_d<4, 128>(a, grid, st);
    else launch_d<4, 256>(a, grid, st);
  } else {
    if (D == 64) launch_d<8, 64>(a, grid, st);
    else if (D == 128) launch_d<8, 128>(a, grid, st);
    else launch_d<8, 256>(a, grid, st);
  }
  VKV_HIP(hipGetLastError());
  if (a.n_parts > 1) {
    hipLaunchKernelGGL(qdecode_combine_kernel, dim3(static_cast<unsigned>(n_seqs) * a.Hq),
                       dim3(D >= 256 ? 256 : D), 0, st, a, D);
    VKV_HIP(hipGetLastError());
  }
}

}  // namespace vkv
