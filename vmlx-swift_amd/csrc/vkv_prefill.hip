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
// Work layout.  A workgroup of 8 waves (two per SIMD, one workgroup per
// CU) owns a block of 256 query rows of one (row of the batch, kv head) and
// one key range; a query row is one (query head of the group, position),
// position-major.  Wave w owns rows 32w .. 32w + 31.  Each 32-token key tile
// takes two phases separated by workgroup barriers: a matrix phase (the
// scores of the tile, the P.V of the tile before) and a softmax phase.
// Waves 4..7 run one phase behind waves 0..3, so the two waves of a SIMD are
// always in different phases: one wave's MFMAs overlap the other's softmax
// (ping-pong), and the wave in its matrix phase issues at the higher
// priority.  Per tile:
//   * K and V tiles (32 rows of D elements each) go HBM -> LDS with
//     global_load_lds_dwordx4 two tiles ahead into four stages (each wave
//     loads one 1 KB piece of each); the per-lane source offsets place each
//     16-byte piece at its swizzled slot, so the tiles are bank-conflict
//     free with no register staging;
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

constexpr int kTok = 32;      // tokens per key tile
constexpr int kStages = 4;    // K+V tiles in LDS; the open-tile loop is unrolled by it
constexpr int kWaves = 8;     // two per SIMD, one workgroup per CU
constexpr int kThreads = 64 * kWaves;
constexpr float kTau = 8.0f;  // rescale threshold (log2)
constexpr float kLog2e = 1.4426950408889634f;

// Layout for head dim D (keys and values).  Every wave owns 32 query rows.
// Up to 128 dims a wave holds all D output dims, so a workgroup covers 8
// row blocks; at 256 dims the two waves of a SIMD own the same 32 rows and
// split the output dims (each computes the full scores), so a workgroup
// covers 4 row blocks.
template <int D>
struct PfCfg {
  static constexpr int kChunks = D / 16;            // K steps of the score MFMA
  static constexpr int kSplit = D == 256 ? 2 : 1;   // waves sharing a row block
  static constexpr int kDBw = D / 32 / kSplit;      // 32-dim output blocks per wave
  static constexpr int kRB = kWaves / kSplit;       // row blocks per workgroup
  static constexpr int kRows = 32 * kRB;            // query rows per workgroup
  static constexpr int kRowB = 2 * D;               // bytes per K / V row
  static constexpr int kTileB = kTok * kRowB;       // bytes per K (or V) tile
  static constexpr int kSlots = D / 8;              // 16-byte pieces per row
  static constexpr int kKLoads = kTileB / 1024;     // 1 KB loads of a K (or V) tile
  static constexpr int kLoads = 2 * kKLoads / kWaves;  // 1 KB loads per wave per tile
  static_assert(D == 64 || D == 128 || D == 256, "head dims 64, 128, 256");
  static_assert(kLoads >= 1 && kLoads * kWaves == 2 * kKLoads, "loads split evenly");
};
// LDS slot of piece p of key row t is p ^ kswz(t): a score read of 16
// consecutive rows at one piece hits 16 distinct 16-byte bank groups (rows
// of 256 or 512 bytes: t & 15; of 128 bytes, where rows t and t + 1 already
// differ by half the banks: (t / 2) & 7).
template <int D>
__device__ __forceinline__ int kswz(int t) {
  return D == 64 ? (t >> 1) & 7 : t & 15;
}
// value rows: piece p at slot p ^ vswz(t & 3), for the transposing reads
// (4 rows x 32 bytes per 16 lanes)
template <int D>
__device__ __forceinline__ int vswz(int t) {
  return D == 64 ? 2 * ((t >> 1) & 1) : 4 * (t & 3);
}

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
// Before every barrier a wave waits for all of its tile loads but the last
// tile's (LOADS), and for its LDS reads.  The scheduling barriers
// keep the compiler from moving any instruction from one phase into the
// other.
// A wave enters a matrix phase at issue priority 1 and a softmax phase at
// 0, so that on a SIMD the MFMAs of the one wave issue back to back and the
// softmax of the other fills the cycles between them.
template <int PRIO, int LOADS>
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(LOADS) : "memory");
  __builtin_amdgcn_s_setprio(PRIO);
  __builtin_amdgcn_sched_barrier(0);
}
__device__ __forceinline__ void tile_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// A value a phase produces is complete before the phase's closing barrier:
// the compiler may otherwise move pure arithmetic (the exponentials, the
// MFMAs) across the barrier into the other phase.
__device__ __forceinline__ void pin(float v) { asm volatile("" ::"v"(v)); }
__device__ __forceinline__ void pin(const u32x4_t& v) { asm volatile("" ::"v"(v)); }
__device__ __forceinline__ void pin(const f32x16_t& v) { asm volatile("" ::"v"(v)); }
// last visible key of a tile relative to its first, clamped to -1 .. kTok
__device__ __forceinline__ int tile_limit(int64_t last) {
  return static_cast<int>(last < -1 ? -1 : (last > kTok ? kTok : last));
}
// max of a value over the two 32-lane halves of the wave
__device__ __forceinline__ float halves_max(float v) {
  float lo = v, hi = v;
  // lo's upper half <- hi's lower half: lo = the lower half's values in both
  // halves, hi = the upper half's
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
  return fmaxf(lo, hi);
}

// QSEM: the quantized-SDPA arithmetic (KVCache.swift:1909-1997): queries
// times the scale rounded to the dtype, rounded again, instead of fp32 scores
// times the scale; scores rounded to the dtype before the softmax.
template <int DT, bool QSEM, int D>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
prefill_kernel(const AttnArgs a, int rep) {
  using Cfg = PfCfg<D>;
  constexpr int kChunks = Cfg::kChunks, kDBw = Cfg::kDBw, kRows = Cfg::kRows;
  constexpr int kRowB = Cfg::kRowB, kTileB = Cfg::kTileB, kLoads = Cfg::kLoads;
  __shared__ __attribute__((aligned(16))) uint8_t kv[kStages][2][kTileB];  // [stage][K/V]

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // waves w and w + 4 share a SIMD; group 1 runs one phase behind group 0
  const int grp = wave >> 2;
  // the wave's 32-row block and (at 256 dims) half of the output dims
  const int rb = wave % Cfg::kRB, dh = wave / Cfg::kRB;
  const int lane = tid & 63, l32 = lane & 31, kg = lane >> 5;
  // workgroup id -> (kv head, part, row block, row of the batch), kv head
  // fastest: workgroups are dealt to the 8 XCDs in id order, so with 8 kv
  // heads each XCD serves one head, and that head's K/V, re-read by every
  // row block and part, stays in the XCD's L2
  const int L = a.L;
  const int rblocks = static_cast<int>((static_cast<int64_t>(L) * rep + kRows - 1) / kRows);
  // parts of this launch: all, or a window part0 .. part0 + parts_run - 1
  const int prun = a.parts_run > 0 ? a.parts_run : a.n_parts;
  int id = blockIdx.x;
  const int hk = id % a.Hkv;
  id /= a.Hkv;
  const int part = a.part0 + id % prun;
  id /= prun;
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
  // tiles that every row of the workgroup sees whole (no mask work)
  int n_open = 0;
  if (!some_none) {
    const int64_t kmin = a.mask_mode == 1 ? T - L + row0 / rep : T - 1;
    const int64_t open = min<int64_t>(kmin, k_end - 1) - k_begin + 1;
    n_open = open > 0 ? static_cast<int>(min<int64_t>(open / kTok, ntiles)) : 0;
  }

  // ---- this lane's query row and its queries: B operand of score step c
  // = dims 16c + 8 kg .. +8
  using E = Elem<DT>;
  const int64_t qrow = row0 + 32 * rb + l32;
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

  f32x16_t o[kDBw];  // output dims 32 (dh kDBw + db) ..
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
  for (int db = 0; db < kDBw; db++) o[db] = f32x16_t{};

  if (ntiles > 0) {
    // ---- tile loads.  A tile is 2 kKLoads loads of 1 KB (the K tile's,
    // then the V tile's); wave w issues loads w + 8 x.  Lane lam of a load
    // fills LDS slot lam % kSlots of its row (the load covers 1024 / kRowB
    // consecutive rows) with the row's piece (lam % kSlots) ^ swizzle(row).
    // row 0 of the K / V views is token t_base (a window of the keys)
    const uint8_t* kbase = a.kv.kc.ptr + b * a.kv.kc.sb + hk * a.kv.kc.sh;
    const uint8_t* vbase = a.kv.vc.ptr + b * a.kv.vc.sb + hk * a.kv.vc.sh;
    const int64_t kst = a.kv.kc.st, vst = a.kv.vc.st;
    // the lane's row and piece in load x (recomputed where needed: at 256
    // dims four loads' worth would hold registers through the loop)
    auto lrow = [&](int x) __attribute__((always_inline)) {
      return ((wave + kWaves * x) % Cfg::kKLoads) * (1024 / kRowB) + lane / Cfg::kSlots;
    };
    auto lpiece = [&](int x) __attribute__((always_inline)) {
      const int slot = lane % Cfg::kSlots, r = lrow(x);
      return wave + kWaves * x >= Cfg::kKLoads ? slot ^ vswz<D>(r & 3) : slot ^ kswz<D>(r);
    };
    uint32_t loff[kLoads];  // offsets within a whole tile (T * stride < 2^31, host-checked)
#pragma unroll
    for (int x = 0; x < kLoads; x++) {
      const bool is_v = wave + kWaves * x >= Cfg::kKLoads;  // wave-uniform
      loff[x] = static_cast<uint32_t>(lrow(x) * (is_v ? vst : kst)) + 16 * lpiece(x);
    }
    auto load_tile = [&](int i, int s) __attribute__((always_inline)) {
      const int ti = min(i, ntiles - 1);  // clamped: every wave issues the same loads
      const int64_t t0 = k_begin + static_cast<int64_t>(kTok) * ti;
#pragma unroll
      for (int x = 0; x < kLoads; x++) {
        const int n = wave + kWaves * x, pn = n % Cfg::kKLoads;
        const bool is_v = n >= Cfg::kKLoads;
        const int64_t st = is_v ? vst : kst;
        uint32_t off = loff[x];
        if (t0 + kTok > T) {
          // rows past the end repeat the last row (masked); t0 < T here
          const int t = min<int64_t>(lrow(x), T - 1 - t0);
          off = static_cast<uint32_t>(t * st) + 16 * lpiece(x);
        }
        // wave-uniform (M0), which the compiler does not see through the select
        const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_addr(&kv[s][is_v][0]) + 1024 * pn);
        dma16((is_v ? vbase : kbase) + (t0 - a.t_base) * st, off, dst);
      }
    };

    // ---- per-lane LDS addresses
    // score A operand, step c: K row l32, piece 2c + kg at slot (2c + kg) ^ kswz(l32)
    const uint32_t ka = lds_addr(&kv[0][0][0]) + l32 * kRowB;
    const int kx = kswz<D>(l32);
    // value A operand (dim block db, k-step ks, token half hf): lane
    // 16 a4 + 4 e + jj reads V row 16 ks + 8 hf + 4 (a4 / 2) + e, dims
    // 32 db + 16 (a4 % 2) + 4 jj .. +4 = piece 4 db + 2 (a4 % 2) + jj / 2
    const int a4 = lane >> 4, e4 = (lane >> 2) & 3, jj = lane & 3;
    const uint32_t va = lds_addr(&kv[0][1][0]) + (4 * (a4 >> 1) + e4) * kRowB + 8 * (jj & 1);
    const int vpc = 2 * (a4 & 1) + (jj >> 1);  // piece within the 4-piece group
    const int vx = vswz<D>(e4);                // swizzle of rows 4 (a4 / 2) + e (+ 8 hf + 16 ks)

    // QSEM: P carried as hi + lo (two operands of the dtype, ~16
    // significant bits), so the weighted sum keeps fp32-like accuracy on
    // large value channels; otherwise one operand
    u32x4_t pb[2], pl[2];
    f32x16_t x;
    // the matrix phase: scores of the tile at LDS base kb (K rows) into x
    // and, with PV, O^T += V^T P^T for the tile at LDS base vb (V rows).
    // Every LDS read is issued before the first MFMA, so the MFMAs run
    // back to back instead of each waiting for its operand's read.
    auto matrix = [&](uint32_t kb, uint32_t vb, auto PV_) __attribute__((always_inline)) {
      constexpr bool PV = decltype(PV_)::value;
      u32x4_t kf[kChunks];
#pragma unroll
      for (int c = 0; c < kChunks; c++)
        kf[c] = *lds_ptr<const u32x4_t>(kb + 16 * ((2 * c + kg) ^ kx));
      u32x4_t vf[kDBw][2];
      if constexpr (PV) {
#pragma unroll
        for (int db = 0; db < kDBw; db++)
#pragma unroll
          for (int ks = 0; ks < 2; ks++) {
            // rows 16 ks + 8 hf + 4 (a4 / 2) + e (row & 3 = e): piece
            // 4 gdb + vpc (gdb = the global dim block) at slot (4 gdb + vpc) ^ vswz(e)
            const uint32_t slot = 16 * ((4 * (dh * kDBw + db) + vpc) ^ vx);
            const uint32_t off0 = (16 * ks) * kRowB + slot;
            const uint32_t off1 = (16 * ks + 8) * kRowB + slot;
            const i16x4_t x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_ptr<i16x4_t>(vb + off0));
            const i16x4_t x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_ptr<i16x4_t>(vb + off1));
            const u32x2_t w0 = __builtin_bit_cast(u32x2_t, x0), w1 = __builtin_bit_cast(u32x2_t, x1);
            vf[db][ks] = u32x4_t{w0[0], w0[1], w1[0], w1[1]};
          }
      }
      x = f32x16_t{};
      if constexpr (PV) {
        // the score chain (8 dependent MFMAs) interleaved with the P.V
        // MFMAs (one chain per 32-dim block)
        constexpr int kPv = (QSEM ? 4 : 2) * kDBw;  // P.V MFMAs
        sfor<kChunks>([&](auto C) {
          constexpr int c = decltype(C)::value;
          x = mfma<DT>(kf[c], qf[c], x);
          // the P.V MFMAs spread evenly over the score steps
          sfor<kPv>([&](auto J) {
            constexpr int n = decltype(J)::value;  // n-th P.V MFMA
            if constexpr (n >= c * kPv / kChunks && n < (c + 1) * kPv / kChunks) {
              constexpr int db = n % kDBw;
              constexpr int q = n / kDBw;  // QSEM: ks hi, ks lo; else ks
              constexpr int ks = QSEM ? q / 2 : q;
              if constexpr (QSEM && q % 2 == 1)
                o[db] = mfma<DT>(vf[db][ks], pl[ks], o[db]);
              else
                o[db] = mfma<DT>(vf[db][ks], pb[ks], o[db]);
            }
          });
        });
        if constexpr (D <= 128) {
          __builtin_amdgcn_sched_group_barrier(0x100, kChunks + 4 * kDBw, 0);  // LDS reads
          __builtin_amdgcn_sched_group_barrier(0x008, kChunks + kPv, 0);       // MFMAs
        } else {
          // at 256 dims every read at once would not fit the registers:
          // eight rounds of reads, each followed by its share of MFMAs
          sfor<8>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x100, (kChunks + 4 * kDBw) / 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, (kChunks + kPv) / 8, 0);
          });
        }
#pragma unroll
        for (int db = 0; db < kDBw; db++) pin(o[db]);
      } else {
#pragma unroll
        for (int c = 0; c < kChunks; c++) x = mfma<DT>(kf[c], qf[c], x);
        if constexpr (D <= 128) {
          __builtin_amdgcn_sched_group_barrier(0x100, kChunks, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, kChunks, 0);
        } else {
          sfor<4>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x100, kChunks / 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, kChunks / 4, 0);
          });
        }
      }
      pin(x);
    };
    // softmax of the row over tile i's scores x: the running max and sum,
    // the rescale of o, and the P operands.  EDGE: keys past the range or
    // the causal limit of some row are masked
    auto softmax = [&](int i, auto EDGE_) __attribute__((always_inline)) {
      constexpr bool EDGE = decltype(EDGE_)::value;
      const int64_t t0 = k_begin + static_cast<int64_t>(kTok) * i;
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
      if constexpr (EDGE) {
        if (QSEM && some_none && __builtin_amdgcn_ballot_w64(kmax < 0)) {
          // rows that see no key: equal scores (0) on the row's keys
          const bool none = kmax < 0;
          const int lim = tile_limit((none ? k_end - 1 : min<int64_t>(kmax, k_end - 1)) - t0);
#pragma unroll
          for (int j = 0; j < 16; j++) {
            if (none) x[j] = 0.0f;
            if (8 * (j >> 2) + 4 * kg + (j & 3) > lim) x[j] = -INFINITY;
          }
        } else {
          const int lim = tile_limit(min<int64_t>(kmax, k_end - 1) - t0);
#pragma unroll
          for (int j = 0; j < 16; j++)
            if (8 * (j >> 2) + 4 * kg + (j & 3) > lim) x[j] = -INFINITY;
        }
      }
      float mx = x[0];
#pragma unroll
      for (int j = 1; j < 16; j++) mx = fmaxf(mx, x[j]);
      mx = halves_max(mx) * cl;  // scale > 0
      if (__builtin_amdgcn_ballot_w64(mx > m_run + kTau)) {
        const float mn = fmaxf(m_run, mx);
        const float al = fast_exp2f(m_run - mn);
        l_run *= al;
#pragma unroll
        for (int db = 0; db < kDBw; db++) o[db] *= al;
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
          pin(pl[ks]);
        }
        pin(pb[ks]);
      }
      pin(l_run);
    };

    // ---- the tile loop, in two phases per tile separated by workgroup
    // barriers: a matrix phase (loads of tile i + 2, scores of tile i,
    // O += V P of tile i - 1) and a softmax phase (tile i).  Group 1 runs
    // one phase behind group 0, so on each SIMD one wave's MFMAs overlap the
    // other wave's softmax.  Tile i lives in stage i % 4: its K is read in
    // the matrix phases of i, its V in those of i + 1 (the last read, by
    // group 1, ends before the phase in which tile i + 4 is loaded over it).
    // Tiles that every row sees whole run unrolled by the stage count, so
    // every LDS address is a per-lane base plus an immediate offset; the
    // rest (masked) run with the stage computed.
    const uint32_t stage_b = 2 * kTileB;
    load_tile(0, 0);
    load_tile(1, 1);
    phase_barrier<1, kLoads>();
    if (grp) phase_barrier<1, kLoads>();
    load_tile(2, 2);
    matrix(ka, 0, std::false_type{});
    phase_barrier<0, kLoads>();
    // softmax of tile i, then the matrix phase of tile i + 1
    auto open_tile = [&](int i, auto S_) __attribute__((always_inline)) {
      constexpr int S = decltype(S_)::value;
      softmax(i, std::false_type{});
      phase_barrier<1, kLoads>();
      load_tile(i + 3, (S + 3) % kStages);
      // past the last tile this scores the clamped copy of the last tile
      // (loaded and complete like any other): unused, but no branch
      matrix(ka + ((S + 1) % kStages) * stage_b, va + S * stage_b, std::true_type{});
      phase_barrier<0, kLoads>();
    };
    int i = 0;
    for (; i + kStages <= n_open; i += kStages) {
      open_tile(i, std::integral_constant<int, 0>{});
      open_tile(i + 1, std::integral_constant<int, 1>{});
      open_tile(i + 2, std::integral_constant<int, 2>{});
      open_tile(i + 3, std::integral_constant<int, 3>{});
    }
    for (; i < ntiles; i++) {
      const int s = i % kStages;
      if (i < n_open)
        softmax(i, std::false_type{});
      else
        softmax(i, std::true_type{});
      phase_barrier<1, kLoads>();
      load_tile(i + 3, (s + 3) % kStages);
      matrix(ka + ((s + 1) % kStages) * stage_b, va + s * stage_b, std::true_type{});
      phase_barrier<0, kLoads>();
    }
    // group 0 has one barrier fewer: it meets group 1's last one here
    if (!grp) phase_barrier<0, kLoads>();
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
    for (int db = 0; db < kDBw; db++)
#pragma unroll
      for (int m = 0; m < 4; m++) {
        const int d = 32 * (dh * kDBw + db) + 8 * m + 4 * kg;
        u32x2_t w;
        w[0] = pack2<DT>(o[db][4 * m] * inv, o[db][4 * m + 1] * inv);
        w[1] = pack2<DT>(o[db][4 * m + 2] * inv, o[db][4 * m + 3] * inv);
        *reinterpret_cast<u32x2_t*>(op + d) = w;
      }
  } else {
    // unnormalized partial; (max, sum) with the max in natural-log units
    const int64_t base = (grow * a.Hq + h) * a.n_parts + part;
    float* wo = a.ws_o + base * D + 32 * dh * kDBw;
#pragma unroll
    for (int db = 0; db < kDBw; db++)
#pragma unroll
      for (int j = 0; j < 16; j++) wo[32 * db + 8 * (j >> 2) + 4 * kg + (j & 3)] = o[db][j];
    if (kg == 0 && dh == 0) {  // the two dim halves hold the same (max, sum)
      a.ws_ml[base * 2] = lt > 0.f ? m_run * (1.0f / kLog2e) : -INFINITY;
      a.ws_ml[base * 2 + 1] = lt;
    }
  }
}

}  // namespace

bool prefill_supported(int dtype, int bits, const AttnArgs& a) {
  if (bits != 0 || a.kv.table || a.kv.qfmt) return false;
  if (dtype != kBF16 && dtype != kF16) return false;
  if (a.L < 2 || a.Dv != a.D || a.Hq % a.Hkv) return false;
  if (a.D != 64 && a.D != 128 && a.D != 256) return false;
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

static int prefill_rows_per_wg(int D) { return D == 256 ? PfCfg<256>::kRows : PfCfg<128>::kRows; }

int prefill_parts(int64_t rows, int Hkv, int64_t L, int rep, int64_t T, int D, int32_t* part_tokens) {
  const int64_t rpw = prefill_rows_per_wg(D);
  const int64_t rblocks = (L * rep + rpw - 1) / rpw;
  const int64_t wgs = rows * Hkv * rblocks;  // rows = batch rows here
  // one workgroup per CU
  int64_t parts = std::max<int64_t>(1, 256 / std::max<int64_t>(1, wgs));
  parts = std::min<int64_t>(parts, std::max<int64_t>(1, (T + 255) / 256));
  int64_t pt = (T + parts - 1) / parts;
  pt = (pt + kTok - 1) / kTok * kTok;
  *part_tokens = static_cast<int32_t>(std::max<int64_t>(kTok, pt));
  return static_cast<int>((T + *part_tokens - 1) / *part_tokens);
}

template <int D>
static void launch_prefill_d(int dtype, bool qsem, const AttnArgs& a, const dim3& grid, int rep,
                             hipStream_t st) {
  if (dtype == kBF16 && qsem)
    hipLaunchKernelGGL((prefill_kernel<kBF16, true, D>), grid, dim3(kThreads), 0, st, a, rep);
  else if (dtype == kBF16)
    hipLaunchKernelGGL((prefill_kernel<kBF16, false, D>), grid, dim3(kThreads), 0, st, a, rep);
  else if (qsem)
    hipLaunchKernelGGL((prefill_kernel<kF16, true, D>), grid, dim3(kThreads), 0, st, a, rep);
  else
    hipLaunchKernelGGL((prefill_kernel<kF16, false, D>), grid, dim3(kThreads), 0, st, a, rep);
}

void launch_prefill(int dtype, bool qsem, const AttnArgs& a, int64_t batch, hipStream_t st,
                    bool combine) {
  if (batch <= 0 || a.L <= 0) return;
  VKV_CHECK(a.D == 64 || a.D == 128 || a.D == 256, "prefill kernel head dim");
  const int prun = a.parts_run > 0 ? a.parts_run : a.n_parts;
  VKV_CHECK(a.part0 >= 0 && a.part0 + prun <= a.n_parts, "prefill part window");
  const int rep = a.Hq / a.Hkv;
  const int64_t rpw = prefill_rows_per_wg(a.D);
  const int64_t rblocks = (static_cast<int64_t>(a.L) * rep + rpw - 1) / rpw;
  const int64_t wgs = rblocks * prun * a.Hkv * batch;
  VKV_CHECK(wgs < (int64_t{1} << 31), "too many prefill workgroups for one launch");
  const dim3 grid(static_cast<unsigned>(wgs));
  if (a.D == 64)
    launch_prefill_d<64>(dtype, qsem, a, grid, rep, st);
  else if (a.D == 128)
    launch_prefill_d<128>(dtype, qsem, a, grid, rep, st);
  else
    launch_prefill_d<256>(dtype, qsem, a, grid, rep, st);
  VKV_HIP(hipGetLastError());
  if (combine && a.n_parts > 1) launch_attn_combine(dtype, a, batch * a.L, st);
}

}  // namespace vkv
