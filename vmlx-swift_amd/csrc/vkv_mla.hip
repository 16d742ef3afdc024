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
// token split, group of 128 query heads) and walks the split 32 tokens at
// a time, all contractions on v_mfma_f32_32x32x16_bf16:
//   * raw tiles (codes and scale/bias of 32 entries, 19584 contiguous
//     bytes of a page) go from HBM straight into LDS with
//     global_load_lds_dwordx4, three tiles ahead, so no registers hold them;
//   * each thread dequantizes 9 (entry, 8-dim) pieces of the next tile from
//     the raw stage into a bf16 key tile (double buffered), spread over the
//     matrix-core work of the current tile;
//   * scores: wave w computes S^T = K Q^T for heads 32w..32w+31 (A = key
//     rows from LDS, B = the queries: 32 of 36 16-dim chunks in registers,
//     the rope chunks in LDS); lane l then holds head l % 32 for tokens
//     8 (j / 4) + 4 (l / 32) + j % 4, j = 0..15;
//   * softmax against a fixed running max; those 16 probabilities are, in
//     that order, the wave's own A operands of the P.V contraction (k-step
//     ks = tokens 16 ks .. 16 ks + 15, lane l / 32 picking tokens
//     {0-3, 8-11} or {4-7, 12-15} of it), so the wave starts P.V on its own
//     heads from registers while the other waves' probabilities meet in an
//     LDS tile;
//   * P.V: wave w accumulates output dims 128w..128w+127 of all 128 heads
//     (256 fp32 accumulators); B = values read with the transposing LDS
//     load ds_read_b64_tr_b16 (within 16 lanes, lane i receives element
//     i % 4 of the 8 bytes lane 4e + i / 4 addressed: pointing those lanes
//     at 4 consecutive dims of token T + e hands lane i dim i of tokens
//     T .. T + 3, the tokens its probability operand pairs it with).
// Split partials (o / l in bf16, running max, sum) are merged by
// mla_combine_kernel as sdpa_vector_2pass_2 merges them
// (Source/Cmlx/mlx-generated/metal/sdpa_vector.h:320-394).
//
// LDS key tile: row t (entry) = 72 16-byte pieces (piece q = dims 8q..8q+7)
// at slot q ^ kswz(t), kswz(t) = 4 t1 ^ t2 ^ 2 t3 (t_b = bit b of t), rows
// 1152 bytes apart.  The score operand reads (32 rows, two adjacent
// pieces), the transposing value reads (4 rows x 32 bytes per 16 lanes) and
// the dequant stores (2 rows x 8 pieces per 16 lanes) each touch 16
// distinct bank quads per 256 bytes (checked on the CPU against a 64-bank
// model).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <utility>

#include "vkv_device.h"
#include <hip/hip_ext.h>

#include "vkv_internal.h"

namespace vkv {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;

constexpr int kDK = 576;                   // entry dims (latent + rope)
constexpr int kDV = 512;                   // value dims
constexpr int kTile = 32;                  // tokens per tile
constexpr int kHeads = 128;                // query heads per workgroup (32 per wave)
constexpr int kChunks = kDK / 16;          // K steps of the score MFMA
constexpr int kQReg = kDV / 16;            // query chunks held in registers
constexpr int kKRow = kDK * 2;             // bytes per key-tile row
constexpr int kKTile = kTile * kKRow;      // bytes per key tile
constexpr int kSbRow = (kDK / 64) * 4;     // (scale, bias) bytes per entry
constexpr int kRawCodes = kTile * kDK;     // code bytes per raw tile
constexpr int kRawTile = kRawCodes + kTile * kSbRow;  // bytes per raw tile
constexpr int kStages = 3;                 // raw tiles in flight
constexpr int kDmaPerWave = 5;             // 16-byte-per-lane loads per wave per tile
constexpr int kPRow = 80;                  // bytes per head row of the probability tile
constexpr int kQRow = 144;                 // bytes per head row of the rope queries
constexpr int kPieces = 9;                 // dequant pieces per thread per tile
constexpr int kDqQK = 6;                   // of them during the scores, the rest during P.V
constexpr int kKaAhead = 4;                // score operand reads issued this many steps ahead
constexpr int kKaRing = kKaAhead + 1;
constexpr int kMaxSplits = 64;
constexpr float kTau = 64.0f;    // headroom of the fixed running max (log2)
constexpr float kLog2e = 1.4426950408889634f;

// LDS block layout (bytes)
constexpr int kLdsRaw = 0;
constexpr int kLdsKt = kLdsRaw + kStages * kRawTile;
constexpr int kLdsP = kLdsKt + 2 * kKTile;
constexpr int kLdsQ = kLdsP + kHeads * kPRow;
constexpr int kLdsL = kLdsQ + kHeads * kQRow;
constexpr int kLdsFlag = kLdsL + kHeads * 4;
constexpr int kLdsBytes = kLdsFlag + 16;
static_assert(kLdsKt <= 65536, "raw stages below 64 KB");
static_assert(kLdsBytes <= 160 * 1024, "LDS of one workgroup");

static_assert(kRawTile % 16 == 0 && (kRawTile + 1023) / 1024 == 4 * kDmaPerWave,
              "a raw tile is 20 wave-wide 16-byte loads");
static_assert(kTile * (kDK / 8) == 256 * kPieces, "9 pieces per thread");

template <int... Is, class F>
__device__ __forceinline__ void sfor_impl(std::integer_sequence<int, Is...>, F&& f) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void sfor(F&& f) {
  sfor_impl(std::make_integer_sequence<int, N>{}, f);
}

__device__ __forceinline__ f32x16_t mfma(const u32x4_t& a, const u32x4_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// The score contraction's accumulator lives in VGPRs (the 256 AGPRs hold
// the P.V accumulators), which the compiler's MFMA selection does not do on
// its own here, so the score MFMAs are written out: the first with a zero
// accumulator, the rest accumulating in place (back-to-back dependent
// accumulation needs no wait states), and mfma_result_fence pads the wait
// states an XDL result needs before a VALU instruction reads it (at most 19
// for a 16-pass op; 24 here).
__device__ __forceinline__ void mfma_v_first(f32x16_t& c, const u32x4_t& a, const u32x4_t& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_v(f32x16_t& c, const u32x4_t& a, const u32x4_t& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_result_fence(f32x16_t& c) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(c));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// Key-tile slot swizzle of row t.
__device__ __forceinline__ int kswz(int t) {
  return (((t >> 1) & 1) << 2) ^ ((t >> 2) & 1) ^ (((t >> 3) & 1) << 1);
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
// A uniform 32-bit word through the scalar path.
__device__ __forceinline__ int32_t scalar_load(const int32_t* p, int64_t i) {
  return *(reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(
               reinterpret_cast<uintptr_t>(p)) +
           i);
}

// 16 bytes per lane from base + voff to LDS lds + 16 * lane (the wave's
// lanes fill lds .. lds + 1023 in lane order).  Issued as inline assembly
// so the compiler neither waits for these loads at every LDS access nor at
// every barrier: the kernel waits for them itself (vmcnt) before the
// barrier that publishes a raw tile.
__device__ __forceinline__ void dma16(const uint8_t* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, %2" ::"v"(voff), "s"(lds),
               "s"(base)
               : "memory", "m0");
}
// Workgroup barrier for LDS data (LDS ops complete first).  The raw-tile
// loads are waited for separately with raw_wait.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// At most one tile's raw loads (kDmaPerWave) still in flight.
__device__ __forceinline__ void raw_wait_one_tile() {
  asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
}
__device__ __forceinline__ void raw_wait_two_tiles() {
  asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
}
static_assert(kDmaPerWave == 5, "raw_wait_* count 5 loads per tile");
// Keeps memory operations on their side of this point, in the compiler's
// passes and its scheduler, so the interleaving of operand reads, dequant
// and matrix-core steps written below is the one issued.
__device__ __forceinline__ void step_fence() { asm volatile("" ::: "memory"); }

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
mla_kernel(const MlaArgs a) {
  // One LDS block, raw stages first: the raw-tile loads address LDS through
  // M0, and keeping their destinations below 64 KB does not depend on how
  // many M0 bits the load honours.
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
  uint8_t(*raw)[kRawTile] = reinterpret_cast<uint8_t(*)[kRawTile]>(lds + kLdsRaw);
  uint8_t(*kt)[kKTile] = reinterpret_cast<uint8_t(*)[kKTile]>(lds + kLdsKt);
  uint8_t* pt = lds + kLdsP;
  uint8_t* qr = lds + kLdsQ;
  float* lsh = reinterpret_cast<float*>(lds + kLdsL);
  int* restart_flag = reinterpret_cast<int*>(lds + kLdsFlag);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, l32 = lane & 31, kg = lane >> 5;
  const int split = blockIdx.x, b = blockIdx.y;
  const int len = a.seq_lens ? scalar_load(a.seq_lens, b) : a.max_len;
  const int t0 = split * a.split_len;
  const int t1 = min(len, t0 + a.split_len);
  const int ntiles = t1 > t0 ? (t1 - t0 + kTile - 1) / kTile : 0;
  const int hg0 = blockIdx.z * kHeads;        // first head of the workgroup
  const int hw = hg0 + 32 * wave;             // first head this wave scores
  const size_t slot = static_cast<size_t>(b) * a.n_splits + split;

  if (ntiles == 0) {
    const int h = hw + l32;
    if (h < a.H) {
      if (a.n_splits == 1) {
        // an empty sequence yields zeros
        for (int d = kg; d < kDV; d += 2) a.out[b * a.o_ss + h * a.o_sh + d] = 0;
      } else if (kg == 0) {
        a.ws_ml[(slot * a.H + h) * 2] = -INFINITY;
        a.ws_ml[(slot * a.H + h) * 2 + 1] = 0.0f;
      }
    }
    return;
  }

  // ---- queries: chunk c (dims 16c + 8 kg .. +8) of head hw + l32 is the B
  // operand of score step c; chunks 32..35 (rope dims) go to LDS.
  u32x4_t qf[kQReg];
  {
    const int h = min(hw + l32, a.H - 1);
    const uint16_t* qp = a.q + b * a.q_ss + static_cast<int64_t>(h) * a.q_sh + 8 * kg;
#pragma unroll
    for (int c = 0; c < kQReg; c++) qf[c] = *(const g_u32x4_t*)(qp + 16 * c);
#pragma unroll
    for (int c = kQReg; c < kChunks; c++)
      *reinterpret_cast<u32x4_t*>(&qr[(32 * wave + l32) * kQRow + 32 * (c - kQReg) + 16 * kg]) =
          *(const g_u32x4_t*)(qp + 16 * c);
  }
  // the query loads complete here, before the raw-tile loads start (a
  // compiler-inserted wait for them inside the tile loop would also wait
  // for every raw load in flight)
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  const float cl = a.scale * kLog2e;

  // ---- per-lane LDS addresses (the tile buffer and step parts are
  // immediate offsets).  They are recomputed in every tile from an opaque
  // copy of the thread index (a few VALU per tile): kept live across the
  // tile loop they do not fit beside the queries, and the compiler would
  // spill them to scratch, whose reloads wait for every raw-tile load in
  // flight.
  struct LaneAddr {
    uint32_t ka[4];      // score A operand, step c: row l32, piece 2c + kg at
                         // slot 8 (c / 4) + ((2 (c % 4) + kg) ^ kswz(l32))
    uint32_t vb[2][2];   // value B operand [db % 2][token half]
    uint32_t p, qr;      // probability tile / rope queries
    uint32_t dq_code, dq_sb, dq_dst;
    int dt;
  };
  auto lane_addr = [&]() __attribute__((always_inline)) -> LaneAddr {
    int t = tid;
    asm volatile("" : "+v"(t));
    const int ln = t & 63, l2 = ln & 31, g2 = ln >> 5;
    LaneAddr r;
#pragma unroll
    for (int m = 0; m < 4; m++)
      r.ka[m] = lds_addr(&kt[0][0]) + l2 * kKRow + 16 * ((2 * m + g2) ^ kswz(l2));
    // value B operand (dim block db, k-step ks, token half hf): lane
    // 16 a4 + 4 e + jj reads token 16 ks + 8 hf + 4 (a4 / 2) + e, dims
    // 128 wave + 32 db + 16 (a4 % 2) + 4 jj .. +4
    const int a4 = ln >> 4, e = (ln >> 2) & 3, jj = ln & 3;
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int hf = 0; hf < 2; hf++)
        r.vb[u][hf] = lds_addr(&kt[0][0]) + (8 * hf + 4 * (a4 >> 1) + e) * kKRow +
                      16 * (16 * wave + 4 * (u ^ (e >> 1)) + 2 * ((a4 & 1) ^ hf) +
                            ((jj >> 1) ^ (a4 >> 1))) +
                      8 * (jj & 1);
    // probability tile: head row h at h * kPRow, k-step ks at +32 ks, lane
    // half kg at +16 kg (8 bf16 = 8 tokens)
    r.p = lds_addr(&pt[0]) + l2 * kPRow + 16 * g2;
    r.qr = lds_addr(&qr[0]) + (32 * wave + l2) * kQRow + 16 * g2;
    // dequant: thread (entry dt, piece column dj) takes pieces q = 8k + dj
    // (group k).  The chunk format stores piece q of a row at position
    // 18 (q % 4) + q / 4 (qk_word_off), here 18 (dj % 4) + dj / 4 + 2k.
    r.dt = t >> 3;
    const int dj = t & 7;
    r.dq_code = lds_addr(&raw[0][0]) + r.dt * kDK + 8 * (18 * (dj & 3) + (dj >> 2));
    r.dq_sb = lds_addr(&raw[0][0]) + kRawCodes + r.dt * kSbRow;
    r.dq_dst = lds_addr(&kt[0][0]) + r.dt * kKRow + 16 * (dj ^ kswz(r.dt));
    return r;
  };

  // ---- raw tile i (clamped to the last tile, so every wave issues the
  // same number of loads per tile) -> raw stage s: wave w issues the
  // 1024-byte pieces w, w + 4, .., w + 16 of the 20 (18 of codes, 2 of
  // scale/bias; the last holds 128 bytes)
  // page-table entry of tile i (clamped), read through the scalar path one
  // tile before its loads are issued
  auto table_entry = [&](int i) __attribute__((always_inline)) -> int32_t {
    const int ts = t0 + kTile * min(i, ntiles - 1);
    return scalar_load(a.table, static_cast<int64_t>(b) * a.table_stride + ts / a.block_size);
  };
  auto dma_tile = [&](int i, int s, int32_t entry) __attribute__((always_inline)) {
    const int ts = t0 + kTile * min(i, ntiles - 1);
    const int off = ts % a.block_size;
    const uint8_t* chunk = a.base + static_cast<int64_t>(entry) * a.block_bytes;
    const uint8_t* codes = chunk + off * kDK;
    const uint8_t* sbs = chunk + a.sb_off + off * kSbRow;
    const uint32_t dst = lds_addr(&raw[0][0]) + s * kRawTile;
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const uint32_t dma_voff = 16 * ln;
    // pieces wave + 4n, n < 4, are codes; the fifth is code piece 16 or 17
    // (waves 0, 1) or the scale/bias piece 18 or 19 (waves 2, 3)
#pragma unroll
    for (int n = 0; n < kDmaPerWave - 1; n++)
      dma16(codes + 1024 * (wave + 4 * n), dma_voff, dst + 1024 * (wave + 4 * n));
    if (wave < 2) {
      dma16(codes + 1024 * (16 + wave), dma_voff, dst + 1024 * (16 + wave));
    } else if (wave == 2) {
      dma16(sbs, dma_voff, dst + kRawCodes);
    } else if (lane < 8) {
      dma16(sbs + 1024, dma_voff, dst + kRawCodes + 1024);
    }
  };

  // ---- dequant of piece k of tile i: raw stage s -> key buffer nb
  struct Dq {
    u32x2_t c;
    uint32_t sb;
  };
  auto dq_load = [&](const LaneAddr& la, int s, int k, Dq& r) __attribute__((always_inline)) {
    r.c = *lds_ptr<const u32x2_t>(la.dq_code + s * kRawTile + 16 * k);
    r.sb = *lds_ptr<const uint32_t>(la.dq_sb + s * kRawTile + 4 * k);
  };
  // The dequant of a piece runs in 6 parts, one per matrix-core step: a
  // wave overlaps about 4 VALU instructions with each 32-cycle MFMA of its
  // own, and a burst of more stalls the next MFMA.  Part 0 reads the
  // scale/bias, parts 1-4 convert one pair of codes each, part 5 stores
  // the piece.  Each part starts with an empty asm taking its inputs as
  // operands, so its arithmetic cannot be hoisted into an earlier step
  // (and the wait for the piece's LDS reads, issued a piece earlier into
  // the other register set, lands at part 0).
  struct DqOut {
    u32x4_t w;
    float sc, bi;
  };
  auto dq_part = [&](int part, Dq& r, DqOut& o, bool valid, const LaneAddr& la, int nb, int k)
                     __attribute__((always_inline)) {
    if (part == 0) {
      asm volatile("" : "+v"(r.sb));
      const uint32_t sbw = valid ? r.sb : 0u;  // entries past the end dequantize to zeros
      o.sc = __uint_as_float(sbw << 16);
      o.bi = __uint_as_float(sbw & 0xFFFF0000u);
    } else if (part <= 4) {
      const int j = part - 1;  // codes 2j, 2j + 1 of the piece
      // (laundered in place: a copy would cost a move per register)
      asm volatile("" : "+v"(r.c), "+v"(o.sc), "+v"(o.bi));
      const uint32_t x = r.c[j >> 1];
      const int sh = 16 * (j & 1);
      o.w[j] = pack_bf16(fmaf(o.sc, static_cast<float>((x >> sh) & 0xFF), o.bi),
                         fmaf(o.sc, static_cast<float>((x >> (sh + 8)) & 0xFF), o.bi));
    } else {
      asm volatile("" : "+v"(o.w));
      *lds_ptr<u32x4_t>(la.dq_dst + nb * kKTile + 128 * k) = o.w;
    }
  };
  auto dq_store = [&](const LaneAddr& la, Dq& r, bool valid, int nb, int k)
                      __attribute__((always_inline)) {
    DqOut o;
#pragma unroll
    for (int part = 0; part < 6; part++) dq_part(part, r, o, valid, la, nb, k);
  };

  f32x16_t o[4][4];  // [head block (wave + hb) % 4][dim block]: 32 x 32 tiles
  float m_run = -INFINITY, l_run = 0.f, m_est = -INFINITY;

  // ---- one pass over the split.  Returns true when a later score
  // exceeded the running max by more than kTau (the pass must be redone
  // with m_est, the largest score it saw).
  auto run = [&]() __attribute__((always_inline)) -> bool {
#pragma unroll
    for (int hb = 0; hb < 4; hb++)
#pragma unroll
      for (int db = 0; db < 4; db++) o[hb][db] = f32x16_t{};
    m_run = m_est;
    l_run = 0.f;
    bool redo = false;

    // prologue: raw tiles 0..2 in flight, tile 0 dequantized
    dma_tile(0, 0, table_entry(0));
    dma_tile(1, 1, table_entry(1));
    dma_tile(2, 2, table_entry(2));
    int32_t entry_next = table_entry(3);
    raw_wait_two_tiles();
    lds_barrier();
    {
      const LaneAddr la = lane_addr();
      const bool valid = t0 + la.dt < t1;
      Dq r;
#pragma unroll
      for (int k = 0; k < kPieces; k++) {
        dq_load(la, 0, k, r);
        dq_store(la, r, valid, 0, k);
      }
    }
    raw_wait_one_tile();
    lds_barrier();

    // tile i: scores on key buffer i % 2, dequant of tile i + 1 (raw
    // stage (i + 1) % 3) into buffer (i + 1) % 2, raw tile i + 3 into
    // stage i % 3
    auto tile = [&](int i, auto NB) __attribute__((always_inline)) {
      constexpr int nb = decltype(NB)::value;
      const int s_next = (i + 1) % kStages;
      dma_tile(i + 3, i % kStages, entry_next);
      entry_next = table_entry(i + 4);
      // (after the last tile this dequantizes the clamped copy of it into
      // the idle buffer: harmless, and keeps the tile branch-free)
      const LaneAddr la = lane_addr();
      const bool dq_valid = t0 + kTile * (i + 1) + la.dt < t1;

      // -- scores S^T (32 tokens x 32 heads) with 6 dequant pieces
      f32x16_t s;
      u32x4_t ka[kKaRing], qrope[kChunks - kQReg];
      Dq r[2];
      DqOut dqo;
      dq_load(la, s_next, 0, r[0]);
#pragma unroll
      for (int c = 0; c < kKaAhead; c++)
        ka[c] = *lds_ptr<const u32x4_t>(la.ka[c & 3] + nb * kKTile + 128 * (c >> 2));
      sfor<kChunks>([&](auto C) {
        constexpr int c = decltype(C)::value;
        constexpr int cn = c + kKaAhead;
        if constexpr (cn < kChunks)
          ka[cn % kKaRing] =
              *lds_ptr<const u32x4_t>(la.ka[cn & 3] + nb * kKTile + 128 * (cn >> 2));
        if constexpr (cn >= kQReg && cn < kChunks)
          qrope[cn - kQReg] = *lds_ptr<const u32x4_t>(la.qr + 32 * (cn - kQReg));
        if constexpr (c / 6 < kDqQK) {
          constexpr int k = c / 6, part = c % 6;
          if constexpr (part == 0 && k + 1 < kPieces) dq_load(la, s_next, k + 1, r[(k + 1) & 1]);
          dq_part(part, r[k & 1], dqo, dq_valid, la, nb ^ 1, k);
        }
        if constexpr (c == 0)
          mfma_v_first(s, ka[0], qf[0]);
        else if constexpr (c < kQReg)
          mfma_v(s, ka[c % kKaRing], qf[c]);
        else
          mfma_v(s, ka[c % kKaRing], qrope[c - kQReg]);
        step_fence();
      });

      // -- value operands of this tile (independent of the softmax)
      u32x4_t vb[4][2];
#pragma unroll
      for (int db = 0; db < 4; db++)
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
          const uint32_t off = nb * kKTile + ks * 16 * kKRow + 128 * (db >> 1);
          const i16x4_t x0 =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_ptr<i16x4_t>(la.vb[db & 1][0] + off));
          const i16x4_t x1 =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16(lds_ptr<i16x4_t>(la.vb[db & 1][1] + off));
          const u32x2_t w0 = __builtin_bit_cast(u32x2_t, x0), w1 = __builtin_bit_cast(u32x2_t, x1);
          vb[db][ks] = u32x4_t{w0[0], w0[1], w1[0], w1[1]};
        }

      // -- softmax against the fixed running max; tokens past the end
      // (last tile only) are masked
      mfma_result_fence(s);
      {
        const int rem = t1 - (t0 + kTile * i);
        if (rem < kTile) {
          asm volatile("");  // keep this a branch: one tile in many
#pragma unroll
          for (int j = 0; j < 16; j++)
            if (8 * (j >> 2) + 4 * kg + (j & 3) >= rem) s[j] = -INFINITY;
        }
      }
      // A score above the running max by more than kTau: the first tile
      // takes its max as the running max (nothing is accumulated yet), a
      // later one makes the pass run again.  After the first tile the check
      // runs behind the exponentials, so they overlap the own-head MFMAs
      // (an overflow they may hold is discarded with the pass).
      auto max_check = [&]() __attribute__((always_inline)) {
        float mx = s[0];
#pragma unroll
        for (int j = 1; j < 16; j++) mx = fmaxf(mx, s[j]);
        // scale > 0, so the largest score maps to the largest logit
        const float mloc = mx * cl;
        if (__builtin_amdgcn_ballot_w64(mloc > m_run + kTau)) {
          m_est = fmaxf(m_est, fmaxf(mloc, __shfl_xor(mloc, 32)));
          if (i == 0)
            m_run = m_est;
          else
            redo = true;
        }
      };
      if (i == 0) max_check();
      // -- probabilities of k-step ks, then P.V of the wave's own heads on
      // them from registers while the next k-step's exponentials run
      sfor<2>([&](auto KS) {
        constexpr int ks = decltype(KS)::value;
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
          p[e] = fast_exp2(fmaf(s[8 * ks + e], cl, -m_run));
          l_run += p[e];
        }
        const u32x4_t pw = u32x4_t{pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3]),
                                   pack_bf16(p[4], p[5]), pack_bf16(p[6], p[7])};
        *lds_ptr<u32x4_t>(la.p + wave * 32 * kPRow + 32 * ks) = pw;
#pragma unroll
        for (int db = 0; db < 4; db++) o[0][db] = mfma(pw, vb[db][ks], o[0][db]);
        step_fence();
      });
      if (i != 0) max_check();
      lds_barrier();  // probabilities of every head complete
      // -- P.V on the other waves' heads, with the remaining dequant
      // (the next head block's operands are read one block ahead)
      u32x4_t pa[2][2];
      {
        const uint32_t prow = la.p + ((wave + 1) & 3) * 32 * kPRow;
        pa[0][0] = *lds_ptr<const u32x4_t>(prow);
        pa[0][1] = *lds_ptr<const u32x4_t>(prow + 32);
      }
      sfor<3>([&](auto HB) {
        constexpr int hb = decltype(HB)::value + 1;
        const u32x4_t pa0 = pa[(hb - 1) & 1][0];
        const u32x4_t pa1 = pa[(hb - 1) & 1][1];
        if constexpr (hb < 3) {
          const uint32_t prow = la.p + ((wave + hb + 1) & 3) * 32 * kPRow;
          pa[hb & 1][0] = *lds_ptr<const u32x4_t>(prow);
          pa[hb & 1][1] = *lds_ptr<const u32x4_t>(prow + 32);
        }
        constexpr int k = kDqQK + hb - 1;
        // 8 MFMA steps, dequant parts 0..5 of piece k on the first six
        sfor<8>([&](auto M) {
          constexpr int m = decltype(M)::value;
          if constexpr (m < 6 && k < kPieces) {
            if constexpr (m == 0 && k + 1 < kPieces) dq_load(la, s_next, k + 1, r[(k + 1) & 1]);
            dq_part(m, r[k & 1], dqo, dq_valid, la, nb ^ 1, k);
          }
          o[hb][m & 3] = mfma(m < 4 ? pa0 : pa1, vb[m & 3][m >> 2], o[hb][m & 3]);
          step_fence();
        });
      });
      // next tile's raw stage complete (this wave), then every wave's
      // dequant, P.V reads and raw loads are done
      raw_wait_one_tile();
      lds_barrier();
    };
    static_assert(kDqQK + 3 == kPieces, "the dequant pieces fill the two phases");

    int i = 0;
    for (; i + 1 < ntiles; i += 2) {
      tile(i, std::integral_constant<int, 0>{});
      tile(i + 1, std::integral_constant<int, 1>{});
    }
    if (i < ntiles) tile(i, std::integral_constant<int, 0>{});
    // drain the raw loads issued past the end before the stages are reused
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // total sums of this wave's heads (lanes l and l ^ 32 hold the two
    // token halves), and agreement on a second pass
    const float lt = l_run + __shfl_xor(l_run, 32);
    l_run = lt;
    if (kg == 0) lsh[32 * wave + l32] = lt;
    if (lane == 0) restart_flag[wave] = redo ? 1 : 0;
    __syncthreads();
    const u32x4_t f = *reinterpret_cast<const u32x4_t*>(&restart_flag[0]);
    const bool any = (f[0] | f[1] | f[2] | f[3]) != 0;
    __syncthreads();
    return any;
  };
  // (one copy of the tile loop)
#pragma nounroll
  for (int attempt = 0; attempt < 2; attempt++)
    if (!run()) break;

  // ---- finalize: lane (l32, kg) holds, in o[hb][db][r], head row
  // 32 ((wave + hb) % 4) + 8 (r / 4) + 4 kg + r % 4 and dim
  // 128 wave + 32 db + l32.  Whole sequence: the output; a split: its
  // normalized partial (bf16), and (max, sum) from the heads' score wave.
  uint16_t* dst = a.n_splits == 1 ? a.out : a.ws_o;
  const int64_t dss = a.n_splits == 1 ? a.o_ss : static_cast<int64_t>(a.H) * kDV;
  const int64_t dsh = a.n_splits == 1 ? a.o_sh : kDV;
  const int64_t drow = a.n_splits == 1 ? b : static_cast<int64_t>(slot);
#pragma unroll
  for (int hb = 0; hb < 4; hb++) {
    const int hl = 32 * ((wave + hb) & 3);
#pragma unroll
    for (int m = 0; m < 4; m++) {
      const f32x4_t lt = *reinterpret_cast<const f32x4_t*>(&lsh[hl + 8 * m + 4 * kg]);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int h = hg0 + hl + 8 * m + 4 * kg + e;
        const float inv = lt[e] > 0.f ? 1.0f / lt[e] : 0.f;
        if (h < a.H) {
          uint16_t* op = dst + drow * dss + static_cast<int64_t>(h) * dsh + 128 * wave + l32;
#pragma unroll
          for (int db = 0; db < 4; db++) op[32 * db] = f32_to_bf16(o[hb][db][4 * m + e] * inv);
        }
      }
    }
  }
  if (a.n_splits > 1 && kg == 0) {
    const int h = hw + l32;
    if (h < a.H) {
      a.ws_ml[(slot * a.H + h) * 2] = m_run;
      a.ws_ml[(slot * a.H + h) * 2 + 1] = l_run;
    }
  }
}

// Merge of the split partials of one (sequence, head): 128 threads x 4 dims.
// Partial s holds o_s / l_s (bf16) with its max m_s and sum l_s (log2 units).
// The (max, sum) pairs and the partial rows of up to 8 splits are loaded
// before any is used, so a merge costs one memory round trip per 8 splits.
__global__ void __launch_bounds__(128) mla_combine_kernel(const MlaArgs a) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int d = 4 * threadIdx.x;
  const size_t s0 = static_cast<size_t>(b) * a.n_splits;
  float M = -INFINITY, den = 0.f;
  f32x4_t acc{0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < a.n_splits; c += 8) {
    f32x2_t ml[8];
    u32x2_t v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int s = min(c + j, a.n_splits - 1);  // (clamped slots are selected away)
      ml[j] = *reinterpret_cast<const f32x2_t*>(a.ws_ml + ((s0 + s) * a.H + h) * 2);
      v[j] = *reinterpret_cast<const u32x2_t*>(a.ws_o + ((s0 + s) * a.H + h) * kDV + d);
    }
    float Mc = M;
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (c + j < a.n_splits && ml[j][1] > 0.f) Mc = fmaxf(Mc, ml[j][0]);
    // rescale what the earlier chunks accumulated to the new max
    const float r = Mc == -INFINITY ? 0.f : fast_exp2(M - Mc);
    den *= r;
#pragma unroll
    for (int e = 0; e < 4; e++) acc[e] *= r;
    M = Mc;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float l = ml[j][1];
      if (c + j < a.n_splits && l > 0.f) {
        const float w = fast_exp2(ml[j][0] - M) * l;
        den += w;
        acc[0] = fmaf(w, __uint_as_float(v[j][0] << 16), acc[0]);
        acc[1] = fmaf(w, __uint_as_float(v[j][0] & 0xFFFF0000u), acc[1]);
        acc[2] = fmaf(w, __uint_as_float(v[j][1] << 16), acc[2]);
        acc[3] = fmaf(w, __uint_as_float(v[j][1] & 0xFFFF0000u), acc[3]);
      }
    }
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

bool mla_layout_supported(const uint8_t* base, int64_t block_bytes, int64_t sb_off) {
  // raw tiles are copied with 16-byte loads
  return reinterpret_cast<uintptr_t>(base) % 16 == 0 && block_bytes % 16 == 0 && sb_off % 16 == 0;
}

size_t mla_plan(MlaArgs& a, int want) {
  const int groups = (a.H + kHeads - 1) / kHeads;
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
  const dim3 grid(a.n_splits, a.n_seqs, (a.H + kHeads - 1) / kHeads);
  const TimedLaunch tl = timing_prepare(kTimeMla);
  hipExtLaunchKernelGGL(mla_kernel, grid, dim3(256), 0, st, tl.start, tl.stop, 0, a);
  VKV_HIP(hipGetLastError());
  timing_commit(tl);
  if (a.n_splits > 1) {
    hipLaunchKernelGGL(mla_combine_kernel, dim3(a.H, a.n_seqs), dim3(128), 0, st, a);
    VKV_HIP(hipGetLastError());
  }
}

}  // namespace vkv
