// vkv_prefill.hip -- multi-query attention (L >= 2 query tokens per row:
// chunked prefill) over dense float K/V on gfx950 matrix cores.
//
// Semantics: MLXFast.scaledDotProductAttention with a causal or no mask
// (MLXFast.swift:173-218; causal = query l of L sees keys 0 .. T - L + l,
// with T each row's own length when the rows are ragged: the chunk of a
// continuous batch over a paged pool),
// and quantizedScaledDotProductAttention (KVCache.swift:1909-1997) of the
// quantized caches after their pages are gathered to bf16 (the dequantized
// values the reference's dequantize produces).  Scores and the weighted sum
// accumulate in fp32; the probabilities enter the second contraction as the
// input dtype (bf16 / f16).  Split partials are merged by
// attn_combine_kernel as sdpa_vector_2pass_2 merges them
// (sdpa_vector.h:320-394).
//
// Work layout.  A workgroup of 4 waves (one per SIMD) owns a block of 128
// query rows of one (row of the batch, kv head) and one key range; a query
// row is one (query head of the group, position), position-major.  Wave w
// owns rows 32w .. 32w + 31.  Two workgroups share a CU, so each SIMD runs
// two waves of different workgroups, whose barriers are independent: one
// wave's softmax overlaps the other's matrix-core work.  Per 32-token key
// tile:
//   * K and V tiles (32 rows of D elements each) go HBM -> LDS with
//     global_load_lds_dwordx4 two tiles ahead (each wave loads two 1 KB
//     pieces of each); the per-lane source offsets
//     place each 16-byte piece at its swizzled slot, so the tiles are
//     bank-conflict free with no register staging;
//   * scores S^T = K Q^T on v_mfma_f32_32x32x16 (A = key rows from LDS,
//     B = the wave's queries, in registers): lane l holds query row l % 32
//     of its block for tokens 8 (j / 4) + 4 (l / 32) + j % 4, j = 0..15;
//   * online softmax per row in the lane that owns it (the other token half
//     is lane l ^ 32); a rescale of the accumulators only when a row's max
//     grows by more than 2^kTau;
//   * O^T += V^T P^T: B = the lane's own probabilities, which are exactly
//     the B operand of the k-steps of 16 tokens, A = value columns read with
//     the transposing LDS load ds_read_b64_tr_b16.  O^T keeps one query row
//     per lane, so the rescale and the final 1 / sum need no exchange.
//
// LDS tiles (D = 128: 256-byte rows, 16 slots of 16 bytes): key row t holds
// its piece s at slot s ^ (t & 15) (the score reads of 16 consecutive rows
// hit 16 distinct slots); value row t holds piece s at slot s ^ (4 (t & 3))
// (the transposing reads: 4 rows x 32 bytes per 16 lanes, 16 distinct
// slots per 256 bytes).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <utility>

#include "vkv_device.h"
#include "vkv_internal.h"

namespace vkv {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;

constexpr int kD = 128;                // head dim (keys and values)
constexpr int kTok = 32;               // tokens per key tile
constexpr int kRowB = kD * 2;          // bytes per K / V row
constexpr int kTileB = kTok * kRowB;   // bytes per K (or V) tile
constexpr int kStages = 3;             // K+V tiles in LDS (two in flight); the tile loop is unrolled by it
constexpr int kRows = 128;             // query rows per workgroup
constexpr int kWaves = kRows / 32;     // one 32-row block per wave, one wave per SIMD;
constexpr int kThreads = 64 * kWaves;  // two workgroups per CU
constexpr int kChunks = kD / 16;       // K steps of the score MFMA
constexpr int kDB = kD / 32;           // 32-dim blocks of the output
constexpr int kLoadsPerWave = 2 * kTileB / 1024 / kWaves;  // 16-byte-per-lane loads per wave per tile
constexpr float kTau = 8.0f;           // rescale threshold (log2)
constexpr float kLog2e = 1.4426950408889634f;
static_assert(kLoadsPerWave == 4, "a wave loads two 1 KB pieces of the K tile and two of the V tile");

template <int... Is, class F>
__device__ __forceinline__ void sfor_impl(std::integer_sequence<int, Is...>, F&& f) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void sfor(F&& f) {
  sfor_impl(std::make_integer_sequence<int, N>{}, f);
}

template <int DT>
__device__ __forceinline__ f32x16_t mfma(const u32x4_t& a, const u32x4_t& b, const f32x16_t& c) {
  if constexpr (DT == kBF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (DT == kBF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
}

__device__ __forceinline__ float fast_exp2f(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}
template <class T>
__device__ __forceinline__ __attribute__((address_space(3))) T* lds_ptr(uint32_t a) {
  return reinterpret_cast<__attribute__((address_space(3))) T*>(static_cast<uintptr_t>(a));
}
// 16 bytes per lane from base + voff to LDS lds + 16 * lane; waited for by
// the kernel itself (vmcnt), so the compiler inserts no waits for it.
__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, %2" ::"v"(voff), "s"(lds),
               "s"(base)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// At most one tile's loads (kLoadsPerWave) in flight.
__device__ __forceinline__ void tile_wait_one() { asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); }
__device__ __forceinline__ void tile_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// QSEM: the quantized-SDPA arithmetic (KVCache.swift:1909-1997): queries
// times the scale rounded to the dtype, rounded again, instead of fp32 scores
// times the scale; scores rounded to the dtype before the softmax.
template <int DT, bool QSEM>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
prefill_kernel(const AttnArgs a, int rep) {
  __shared__ __attribute__((aligned(16))) uint8_t kv[kStages][2][kTileB];  // [stage][K/V]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, l32 = lane & 31, kg = lane >> 5;
  // workgroup id -> (kv head, part, row block, row of the batch), kv head
  // fastest: workgroups are dealt to the 8 XCDs in id order, so with 8 kv
  // heads each XCD serves one head, and that head's K/V, re-read by every
  // row block and part, stays in the XCD's L2
  const int L = a.L;
  const int rblocks = static_cast<int>((static_cast<int64_t>(L) * rep + kRows - 1) / kRows);
  int id = blockIdx.x;
  const int hk = id % a.Hkv;
  id /= a.Hkv;
  const int part = id % a.n_parts;
  id /= a.n_parts;
  const int rblk = id % rblocks;
  const int64_t b = id / rblocks;
  // keys of this row of the batch: its own length when the rows are ragged
  // (query l of a row of length T sees keys up to T - L + l when causal)
  const int64_t T = a.kv.seq_lens ? min<int64_t>(a.kv.seq_lens[b], a.kv.T) : a.kv.T;
  const int64_t nrows = static_cast<int64_t>(L) * rep;  // query rows of (b, hk)
  const int64_t row0 = static_cast<int64_t>(rblk) * kRows;
  // keys of this workgroup: the part's range, and for a causal mask the
  // range its last position can see
  const int64_t rlast = min<int64_t>(nrows, row0 + kRows) - 1;
  int64_t k_end = min<int64_t>(T, static_cast<int64_t>(part + 1) * a.part_tokens);
  // QSEM: a query that sees no key (a ragged row shorter than the chunk)
  // has every score at T's lowest value in the reference (where(mask, s,
  // finfo.min)), i.e. uniform weights over all of the row's keys; a
  // workgroup holding such a query scans them all
  const bool some_none = QSEM && a.mask_mode == 1 && T - L + row0 / rep < 0;
  if (a.mask_mode == 1 && !some_none) k_end = min<int64_t>(k_end, T - L + rlast / rep + 1);
  const int64_t k_begin = static_cast<int64_t>(part) * a.part_tokens;
  const int ntiles = k_end > k_begin ? static_cast<int>((k_end - k_begin + kTok - 1) / kTok) : 0;

  // ---- this lane's query row and its queries: B operand of score step c
  // = dims 16c + 8 kg .. +8
  using E = Elem<DT>;
  const int64_t qrow = row0 + 32 * wave + l32;
  int64_t kmax;  // last key the row may see
  u32x4_t qf[kChunks];
  {
    const int64_t qr = min<int64_t>(qrow, nrows - 1);
    const int64_t pos = qr / rep;
    const int r = static_cast<int>(qr % rep);
    kmax = a.mask_mode == 1 ? T - L + pos : T - 1;
    const typename E::T* qp = static_cast<const typename E::T*>(a.q) + b * a.q_sb +
                              static_cast<int64_t>(hk * rep + r) * a.q_sh + pos * a.q_sl + 8 * kg;
#pragma unroll
    for (int c = 0; c < kChunks; c++) qf[c] = *(const g_u32x4_t*)(qp + 16 * c);
  }
  if constexpr (QSEM) {
    const float st = round_to<DT>(a.scale);
#pragma unroll
    for (int c = 0; c < kChunks; c++)
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const uint32_t x = qf[c][w];
        qf[c][w] = pack2<DT>(E::to_f32(static_cast<typename E::T>(x & 0xFFFFu)) * st,
                             E::to_f32(static_cast<typename E::T>(x >> 16)) * st);
      }
  }
  // the query loads complete before the tile loads start (a compiler wait
  // for them inside the tile loop would also wait for every tile load)
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  const float cl = QSEM ? kLog2e : a.scale * kLog2e;

  f32x16_t o[kDB];
  float m_run = -1e30f;  // finite: a masked score (-inf) gives p = 0
  float l_run = 0.f;
  // an attention sink (MLXFast semantics only) is one more logit with a
  // zero value row, counted once per row (sdpa_vector.h:93-96): the running
  // max (log2 units) starts at it with sum 1
  if (!QSEM && a.sinks && part == 0) {
    const int64_t qr = min<int64_t>(qrow, nrows - 1);
    m_run = load_as<DT>(a.sinks, a.sinks_dtype, hk * rep + static_cast<int>(qr % rep)) * kLog2e;
    l_run = kg == 0 ? 1.f : 0.f;  // the two lane halves' sums are added at the end
  }
#pragma unroll
  for (int db = 0; db < kDB; db++) o[db] = f32x16_t{};

  if (ntiles > 0) {
    // ---- tile loads.  Load n (0..7) of a K or V tile fills its rows
    // 4n .. 4n + 3; wave w issues loads w and w + 4 of each.  Lane lam of a load
    // fills LDS slot lam % 16 of row 4n + lam / 16 with the row's piece
    // (lam % 16) ^ swizzle(row).
    const uint8_t* kbase = a.kv.kc.ptr + b * a.kv.kc.sb + hk * a.kv.kc.sh;
    const uint8_t* vbase = a.kv.vc.ptr + b * a.kv.vc.sb + hk * a.kv.vc.sh;
    const int64_t kst = a.kv.kc.st, vst = a.kv.vc.st;
    // per-lane row and slot of this wave's loads (n = wave + kWaves x)
    constexpr int kLx = kLoadsPerWave / 2;
    int lrow[kLx], kpiece[kLx], vpiece[kLx];
#pragma unroll
    for (int x = 0; x < kLx; x++) {
      lrow[x] = 4 * (wave + kWaves * x) + (lane >> 4);
      kpiece[x] = (lane & 15) ^ (lrow[x] & 15);
      vpiece[x] = (lane & 15) ^ (4 * (lrow[x] & 3));
    }
    auto load_tile = [&](int i, int s) __attribute__((always_inline)) {
      const int ti = min(i, ntiles - 1);  // clamped: every wave issues the same loads
      const int64_t t0 = k_begin + static_cast<int64_t>(kTok) * ti;
      const uint32_t kdst = lds_addr(&kv[s][0][0]), vdst = lds_addr(&kv[s][1][0]);
#pragma unroll
      for (int x = 0; x < kLx; x++) {
        // rows past the end repeat the last row (masked); t0 < T here
        const int64_t t = min<int64_t>(t0 + lrow[x], T - 1) - t0;
        const uint32_t koff = static_cast<uint32_t>(t * kst) + 16 * kpiece[x];
        const uint32_t voff = static_cast<uint32_t>(t * vst) + 16 * vpiece[x];
        dma16(kbase + t0 * kst, koff, kdst + 1024 * (wave + kWaves * x));
        dma16(vbase + t0 * vst, voff, vdst + 1024 * (wave + kWaves * x));
      }
    };

    // ---- per-lane LDS addresses
    // score A operand, step c: K row l32, piece 2c + kg at slot (2c + kg) ^ (l32 & 15)
    const uint32_t ka = lds_addr(&kv[0][0][0]) + l32 * kRowB;
    const int kx = l32 & 15;
    // value A operand (dim block db, k-step ks, token half hf): lane
    // 16 a4 + 4 e + jj reads V row 16 ks + 8 hf + 4 (a4 / 2) + e, dims
    // 32 db + 16 (a4 % 2) + 4 jj .. +4 = piece 4 db + 2 (a4 % 2) + jj / 2
    const int a4 = lane >> 4, e4 = (lane >> 2) & 3, jj = lane & 3;
    const uint32_t va = lds_addr(&kv[0][1][0]) + (4 * (a4 >> 1) + e4) * kRowB + 8 * (jj & 1);
    const int vpc = 2 * (a4 & 1) + (jj >> 1);  // piece within the 4-piece group
    const int vx = 4 * (e4 & 3);               // swizzle of rows 4 (a4 / 2) + e (+ 8 hf + 16 ks)

    load_tile(0, 0);
    load_tile(1, 1);
    // the loop is unrolled by the stage count, so every LDS address of a
    // tile is a per-lane base plus an immediate offset
    auto step = [&](int i, auto S_) __attribute__((always_inline)) {
      constexpr int S = decltype(S_)::value;
      tile_wait_one();  // tile i (this wave's loads)
      lds_barrier();    // every wave's loads of tile i; stage (i + 2) % 3 free
      load_tile(i + 2, (S + 2) % kStages);
      const int64_t t0 = k_begin + static_cast<int64_t>(kTok) * i;
      const uint32_t kb = ka + S * 2 * kTileB, vb = va + S * 2 * kTileB;

      // -- scores
      f32x16_t x = f32x16_t{};
      u32x4_t kf[2];
      kf[0] = *lds_ptr<const u32x4_t>(kb + 16 * ((kg) ^ kx));
      sfor<kChunks>([&](auto C) {
        constexpr int c = decltype(C)::value;
        if constexpr (c + 1 < kChunks)
          kf[(c + 1) & 1] = *lds_ptr<const u32x4_t>(kb + 16 * ((2 * (c + 1) + kg) ^ kx));
        x = mfma<DT>(kf[c & 1], qf[c], x);
      });

      // -- value operands (independent of the softmax)
      u32x4_t vf[kDB][2];
#pragma unroll
      for (int db = 0; db < kDB; db++)
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
          // rows 16 ks + 8 hf + 4 (a4 / 2) + e (row & 3 = e): piece
          // 4 db + vpc at slot (4 db + vpc) ^ 4e
          const uint32_t slot = 16 * ((4 * db + vpc) ^ vx);
          const uint32_t off0 = (16 * ks) * kRowB + slot;
          const uint32_t off1 = (16 * ks + 8) * kRowB + slot;
          const i16x4_t x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_ptr<i16x4_t>(vb + off0));
          const i16x4_t x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_ptr<i16x4_t>(vb + off1));
          const u32x2_t w0 = __builtin_bit_cast(u32x2_t, x0), w1 = __builtin_bit_cast(u32x2_t, x1);
          vf[db][ks] = u32x4_t{w0[0], w0[1], w1[0], w1[1]};
        }

      // -- softmax of the row (keys past the range / causal limit masked)
      const bool edge = t0 + kTok - 1 > kmax || t0 + kTok > k_end;
      // QSEM: P carried as hi + lo (two operands of the dtype, ~16
      // significant bits), so the weighted sum keeps fp32-like accuracy on
      // large value channels; otherwise one operand
      u32x4_t pb[2], pl[2];
      if constexpr (QSEM) {
        // the scores are stored in the dtype (quantizedMM returns T,
        // KVCache.swift:1945-1949) before the mask and the softmax: the
        // packed hardware conversion (round to nearest even), then back
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
          const uint32_t w = pack2<DT>(x[j], x[j + 1]);
          x[j] = E::to_f32(static_cast<typename E::T>(w & 0xFFFFu));
          x[j + 1] = E::to_f32(static_cast<typename E::T>(w >> 16));
        }
      }
      if (QSEM && some_none && __builtin_amdgcn_ballot_w64(kmax < 0)) {
        // rows that see no key: equal scores (0) on the row's keys
        const bool none = kmax < 0;
        const int64_t lim = (none ? k_end - 1 : min<int64_t>(kmax, k_end - 1)) - t0;
#pragma unroll
        for (int j = 0; j < 16; j++) {
          if (none) x[j] = 0.0f;
          if (8 * (j >> 2) + 4 * kg + (j & 3) > lim) x[j] = -INFINITY;
        }
      } else if (__builtin_amdgcn_ballot_w64(edge)) {
        const int64_t lim = min<int64_t>(kmax, k_end - 1) - t0;
#pragma unroll
        for (int j = 0; j < 16; j++)
          if (8 * (j >> 2) + 4 * kg + (j & 3) > lim) x[j] = -INFINITY;
      }
      float mx = x[0];
#pragma unroll
      for (int j = 1; j < 16; j++) mx = fmaxf(mx, x[j]);
      mx = fmaxf(mx, __shfl_xor(mx, 32)) * cl;  // scale > 0
      if (__builtin_amdgcn_ballot_w64(mx > m_run + kTau)) {
        const float mn = fmaxf(m_run, mx);
        const float al = fast_exp2f(m_run - mn);
        l_run *= al;
#pragma unroll
        for (int db = 0; db < kDB; db++) o[db] *= al;
        m_run = mn;
      }
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; e++) p[e] = fast_exp2f(fmaf(x[8 * ks + e], cl, -m_run));
        // a sum tree instead of a chain of dependent adds
        l_run += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
        pb[ks] = u32x4_t{pack2<DT>(p[0], p[1]), pack2<DT>(p[2], p[3]), pack2<DT>(p[4], p[5]),
                         pack2<DT>(p[6], p[7])};
        if constexpr (QSEM) {
          float r[8];
#pragma unroll
          for (int w = 0; w < 4; w++) {
            const uint32_t hw = pb[ks][w];
            r[2 * w] = p[2 * w] - E::to_f32(static_cast<typename E::T>(hw & 0xFFFFu));
            r[2 * w + 1] = p[2 * w + 1] - E::to_f32(static_cast<typename E::T>(hw >> 16));
          }
          pl[ks] = u32x4_t{pack2<DT>(r[0], r[1]), pack2<DT>(r[2], r[3]), pack2<DT>(r[4], r[5]),
                           pack2<DT>(r[6], r[7])};
        }
      }
      // -- O^T += V^T P^T
#pragma unroll
      for (int ks = 0; ks < 2; ks++)
#pragma unroll
        for (int db = 0; db < kDB; db++) {
          o[db] = mfma<DT>(vf[db][ks], pb[ks], o[db]);
          if constexpr (QSEM) o[db] = mfma<DT>(vf[db][ks], pl[ks], o[db]);
        }
    };
    for (int i = 0; i < ntiles; i += kStages) {
      step(i, std::integral_constant<int, 0>{});
      if (i + 1 < ntiles) step(i + 1, std::integral_constant<int, 1>{});
      if (i + 2 < ntiles) step(i + 2, std::integral_constant<int, 2>{});
    }
    tile_wait_all();  // the clamped loads issued past the end
  }

  // ---- output: lane (l32, kg) holds, in o[db][j], query row qrow and dim
  // 32 db + 8 (j / 4) + 4 kg + j % 4
  const float lt = l_run + __shfl_xor(l_run, 32);
  if (qrow >= nrows) return;
  const int64_t pos = qrow / rep;
  const int h = hk * rep + static_cast<int>(qrow % rep);
  const int64_t grow = b * L + pos;  // row of the batch x L
  if (a.n_parts == 1) {
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    typename E::T* op = static_cast<typename E::T*>(a.out) + b * a.o_sb + h * a.o_sh + pos * a.o_sl;
#pragma unroll
    for (int db = 0; db < kDB; db++)
#pragma unroll
      for (int m = 0; m < 4; m++) {
        const int d = 32 * db + 8 * m + 4 * kg;
        u32x2_t w;
        w[0] = pack2<DT>(o[db][4 * m] * inv, o[db][4 * m + 1] * inv);
        w[1] = pack2<DT>(o[db][4 * m + 2] * inv, o[db][4 * m + 3] * inv);
        *reinterpret_cast<u32x2_t*>(op + d) = w;
      }
  } else {
    // unnormalized partial; (max, sum) with the max in natural-log units
    const int64_t base = (grow * a.Hq + h) * a.n_parts + part;
    float* wo = a.ws_o + base * kD;
#pragma unroll
    for (int db = 0; db < kDB; db++)
#pragma unroll
      for (int j = 0; j < 16; j++) wo[32 * db + 8 * (j >> 2) + 4 * kg + (j & 3)] = o[db][j];
    if (kg == 0) {
      a.ws_ml[base * 2] = lt > 0.f ? m_run * (1.0f / kLog2e) : -INFINITY;
      a.ws_ml[base * 2 + 1] = lt;
    }
  }
}

}  // namespace

bool prefill_supported(int dtype, int bits, const AttnArgs& a) {
  if (bits != 0 || a.kv.table || a.kv.qfmt) return false;
  if (dtype != kBF16 && dtype != kF16) return false;
  if (a.L < 2 || a.D != kD || a.Dv != kD || a.Hq % a.Hkv) return false;
  if (a.mask_mode != 0 && a.mask_mode != 1) return false;
  // uniform rows: a causal chunk longer than the keys is the generic
  // kernel's; ragged rows (seq_lens) shorter than the chunk see no keys for
  // their first queries, as there
  if (a.mask_mode == 1 && !a.kv.seq_lens && a.L > a.kv.T) return false;
  // 16-byte loads of query rows and of K / V rows
  auto al = [](const void* p, int64_t s0, int64_t s1, int64_t s2) {
    return reinterpret_cast<uintptr_t>(p) % 16 == 0 && s0 % 16 == 0 && s1 % 16 == 0 && s2 % 16 == 0;
  };
  if (!al(a.kv.kc.ptr, a.kv.kc.sb, a.kv.kc.sh, a.kv.kc.st) ||
      !al(a.kv.vc.ptr, a.kv.vc.sb, a.kv.vc.sh, a.kv.vc.st))
    return false;
  const int64_t es = 2;
  if (reinterpret_cast<uintptr_t>(a.q) % 16 || (a.q_sb * es) % 16 || (a.q_sh * es) % 16 ||
      (a.q_sl * es) % 16)
    return false;
  // 8-byte output stores
  if (reinterpret_cast<uintptr_t>(a.out) % 8 || (a.o_sb * es) % 8 || (a.o_sh * es) % 8 ||
      (a.o_sl * es) % 8)
    return false;
  // 32-bit per-lane offsets within a (row, head) of K / V
  if (a.kv.T * std::max(a.kv.kc.st, a.kv.vc.st) >= (int64_t(1) << 31)) return false;
  return true;
}

int prefill_parts(int64_t rows, int Hkv, int64_t L, int rep, int64_t T, int32_t* part_tokens) {
  const int64_t rblocks = (L * rep + kRows - 1) / kRows;
  const int64_t wgs = rows * Hkv * rblocks;  // rows = batch rows here
  // two workgroups per CU
  int64_t parts = std::max<int64_t>(1, 512 / std::max<int64_t>(1, wgs));
  parts = std::min<int64_t>(parts, std::max<int64_t>(1, (T + 255) / 256));
  int64_t pt = (T + parts - 1) / parts;
  pt = (pt + kTok - 1) / kTok * kTok;
  *part_tokens = static_cast<int32_t>(std::max<int64_t>(kTok, pt));
  return static_cast<int>((T + *part_tokens - 1) / *part_tokens);
}

void launch_prefill(int dtype, bool qsem, const AttnArgs& a, int64_t batch, hipStream_t st) {
  if (batch <= 0 || a.L <= 0) return;
  const int rep = a.Hq / a.Hkv;
  const int64_t rblocks = (static_cast<int64_t>(a.L) * rep + kRows - 1) / kRows;
  const int64_t wgs = rblocks * a.n_parts * a.Hkv * batch;
  VKV_CHECK(wgs < (int64_t{1} << 31), "too many prefill workgroups for one launch");
  const dim3 grid(static_cast<unsigned>(wgs));
  if (dtype == kBF16 && qsem)
    hipLaunchKernelGGL((prefill_kernel<kBF16, true>), grid, dim3(kThreads), 0, st, a, rep);
  else if (dtype == kBF16)
    hipLaunchKernelGGL((prefill_kernel<kBF16, false>), grid, dim3(kThreads), 0, st, a, rep);
  else if (qsem)
    hipLaunchKernelGGL((prefill_kernel<kF16, true>), grid, dim3(kThreads), 0, st, a, rep);
  else
    hipLaunchKernelGGL((prefill_kernel<kF16, false>), grid, dim3(kThreads), 0, st, a, rep);
  VKV_HIP(hipGetLastError());
  if (a.n_parts > 1) launch_attn_combine(dtype, a, batch * a.L, st);
}

}  // namespace vkv
