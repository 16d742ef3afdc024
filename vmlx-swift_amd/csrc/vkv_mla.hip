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
constexpr int kStages = 2;                // raw staging buffers
constexpr int kKeyBufs = 3;               // bf16 key tiles (PV, QK, dequant target)
constexpr bool kSoftmaxInPV = false;      // spread the next tile's softmax over P.V
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
  __shared__ __attribute__((aligned(16))) uint16_t kt[kKeyBufs][kTile * kRow];
  __shared__ __attribute__((aligned(16))) int restart_flag[4];
  __shared__ __attribute__((aligned(16))) uint8_t zero_sb[kSbRow + 12];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, n = lane & 15, g = lane >> 4;
  const int split = blockIdx.x, b = blockIdx.y;
  const int len =
      a.seq_lens ? *(reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(
                       reinterpret_cast<uintptr_t>(a.seq_lens)) +
                   b)
                 : a.max_len;
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

  // ---- raw tile loads.  chunk_of(i) is the (block, kv head 0) chunk that
  // holds tile i (tiles past the end reload the last one); issue(i, chunk)
  // puts tile i's code bytes and scale/bias bytes into raw[i % 2].  Wave w
  // issues loads w, w+4, ..., w+16 of the 20: 18 x 1 KB of codes, then the
  // scale/bias bytes, whose 128-byte tail is loaded by 8 lanes while the
  // other 56 re-read byte 0 into the landing pad.
  auto tile_off = [&](int i) __attribute__((always_inline)) {  // token offset of tile i within its block
    const int ts = t0 + kTile * min(i, ntiles - 1);
    return ts % a.block_size;
  };
  // (the table is read through the scalar path: a vector load here would
  // make the compiler wait for every tile load in flight before using it)
  auto chunk_of = [&](int i) __attribute__((always_inline)) {
    const int ts = t0 + kTile * min(i, ntiles - 1);
    const int64_t idx = static_cast<int64_t>(b) * a.table_stride + ts / a.block_size;
    const int32_t blk = *(reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(
                            reinterpret_cast<uintptr_t>(a.table)) +
                        idx);
    return a.base + static_cast<int64_t>(blk) * a.block_bytes;
  };
  auto issue = [&](int i, const uint8_t* chunk) __attribute__((always_inline)) {
    const int off = tile_off(i);
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
      dma16(sb + (lane < 8 ? 1024 + 16 * lane : 0), lds + kRawCodes + 1024);
    }
  };

  // ---- dequant pieces of this thread: token tk, octet residue r = q % 4
  // and parity h, pieces j = 0..8 = dims 8q..8q+7 with q = 8j + 4h + r.
  // The chunk format stores octet q at position (q % 4) * 18 + q / 4 of a
  // token row, so piece j reads position 18r + 2j + h, scale/bias group j,
  // and writes LDS dims 8q: every offset is a lane base plus 16j / 4j / 64j.
  // A 16-lane group holds tokens t and t + 8 x 4 residues x 2 parities,
  // which keeps its 16-byte LDS stores on 16 distinct bank quads.
  const int pr = tid & 3, ph = (tid >> 2) & 1, g16 = tid >> 4;
  const int tk = (g16 & 7) + 16 * (g16 >> 3) + 8 * ((tid >> 3) & 1);
  const int raw_off = tk * kDK + 144 * pr + 8 * ph;  // bytes within a raw tile
  const int sb_off = kRawCodes + tk * kSbRow;         // bytes within a raw tile
  const int kt_off = tk * kRow + 32 * ph + 8 * pr;    // bf16 within a key tile
  struct Piece {
    u32x2_t c;
    uint32_t sb;
  };
  // sbp = scale/bias row of the token (the zero row for tokens past the end)
  auto piece_read = [&](const uint8_t* rc, const uint8_t* sbp, int j) __attribute__((always_inline)) {
    Piece pc;
    pc.c = *reinterpret_cast<const u32x2_t*>(rc + 16 * j);
    pc.sb = *reinterpret_cast<const uint32_t*>(sbp + 4 * j);
    return pc;
  };
  auto piece_write = [&](const Piece& pc, uint16_t* dst, int j) __attribute__((always_inline)) {
    const float s = __uint_as_float(pc.sb << 16), bb = __uint_as_float(pc.sb & 0xFFFF0000u);
    u32x4_t w;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t x = pc.c[h];
      w[2 * h] = pack_bf16(fmaf(s, static_cast<float>(x & 0xFF), bb),
                           fmaf(s, static_cast<float>((x >> 8) & 0xFF), bb));
      w[2 * h + 1] = pack_bf16(fmaf(s, static_cast<float>((x >> 16) & 0xFF), bb),
                               fmaf(s, static_cast<float>(x >> 24), bb));
    }
    *reinterpret_cast<u32x4_t*>(dst + 64 * j) = w;
  };
  // tile i: raw[i % 2] -> kt[i % 3]
  // (ob: an opaque zero that keeps the per-buffer addresses from being
  // hoisted out of the tile loop and held in registers)
  auto piece_src = [&](int i, int ob, const uint8_t*& rc, const uint8_t*& sbp,
                       uint16_t*& dst) __attribute__((always_inline)) {
    const uint8_t* r = &raw[i & (kStages - 1)][0];
    rc = r + raw_off + ob;
    sbp = (t0 + kTile * i + tk < t1) ? r + sb_off + ob : zero_sb;
    dst = &kt[i % kKeyBufs][kt_off + ob];
  };
  auto dequant_all = [&](int i) __attribute__((always_inline)) {
    const uint8_t *rc, *sbp;
    uint16_t* dst;
    piece_src(i, 0, rc, sbp, dst);
    sfor<kPieces>([&](auto J) { piece_write(piece_read(rc, sbp, J), dst, J); });
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

  // ---- scores S^T [32 tokens x 16*HB heads] of tile j (kt[j % 3]), with
  // tile j+1's dequant (raw[(j+1) % 2] -> kt[(j+1) % 3]) interleaved: piece
  // k's LDS reads one step before its stores
  f32x4_t s[2][HB];
  auto qk_dequant = [&](int j, int ob) __attribute__((always_inline)) {
    const uint16_t* K = &kt[j % kKeyBufs][0];
    const uint8_t *rcn, *sbn;
    uint16_t* dn;
    piece_src(j + 1, ob, rcn, sbn, dn);
    const uint16_t* kr0 = K + n * kRow + 8 * g + ob;
    const uint16_t* kr1 = kr0 + 16 * kRow;
#pragma unroll
    for (int tb = 0; tb < 2; tb++)
#pragma unroll
      for (int hb = 0; hb < HB; hb++) s[tb][hb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    u32x4_t ka[2][2];
    ka[0][0] = *reinterpret_cast<const u32x4_t*>(kr0);
    ka[0][1] = *reinterpret_cast<const u32x4_t*>(kr1);
    Piece pc[2];
    pc[0] = piece_read(rcn, sbn, 0);
    sfor<kChunks>([&](auto C) {
      constexpr int c = decltype(C)::value;
      if constexpr (c + 1 < kChunks) {
        ka[(c + 1) & 1][0] = *reinterpret_cast<const u32x4_t*>(kr0 + 32 * (c + 1));
        ka[(c + 1) & 1][1] = *reinterpret_cast<const u32x4_t*>(kr1 + 32 * (c + 1));
      }
      if constexpr (c % 2 == 0 && c / 2 + 1 < kPieces)
        pc[(c / 2 + 1) & 1] = piece_read(rcn, sbn, c / 2 + 1);
      if constexpr (c % 2 == 1) piece_write(pc[(c / 2) & 1], dn, c / 2);
#pragma unroll
      for (int hb = 0; hb < HB; hb++) {
        s[0][hb] = mfma(ka[c & 1][0], qf[hb][c], s[0][hb]);
        s[1][hb] = mfma(ka[c & 1][1], qf[hb][c], s[1][hb]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // ---- softmax of tile j, part 1: mask the tokens past the end (last
  // tile only), check the scores against the fixed running max.  Returns
  // true when the split must be run again.
  auto softmax_check = [&](int j, int ob) __attribute__((always_inline)) {
    const int rem = t1 - (t0 + kTile * j);
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
      if (j == 0) {
        // nothing accumulated yet: take the max as is
#pragma unroll
        for (int hb = 0; hb < HB; hb++) m_run[hb] = m_est[hb];
      } else {
        redo = true;
      }
    }
    return redo;
  };
  // part 2, one (tb, hb) quarter at a time: probabilities of the lane's 4
  // tokens, summed into l_run and packed into the P.V operand
  auto softmax_part = [&](int tb, int hb, u32x4_t (&pn)[HB]) __attribute__((always_inline)) {
    float p[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      p[e] = fast_exp2(fmaf(s[tb][hb][e], cl, -m_run[hb]));
      l_run[hb] += p[e];
    }
    pn[hb][2 * tb] = pack_bf16(p[0], p[1]);
    pn[hb][2 * tb + 1] = pack_bf16(p[2], p[3]);
  };

  // ---- P V of tile i (kt[i % 3], probabilities p) with tile j = i+1's
  // probabilities computed in between (into pn).  Value operand of dim
  // 16 db + n: tokens 4g..4g+3 and 16+4g..16+4g+3 (two transposing reads),
  // two output tiles ahead.
  auto pv_softmax = [&](int i, int ob, const u32x4_t (&p)[HB], u32x4_t (&pn)[HB])
                        __attribute__((always_inline)) {
    // vr0 is made opaque so that the 64 read addresses below are formed
    // from it inside the loop instead of being hoisted out of it and held
    // in (spilled) registers
    uint32_t vr0 = lds_addr(&kt[i % kKeyBufs][(4 * g + (n >> 2)) * kRow + 4 * (n & 3) + ob]);
    asm volatile("" : "+v"(vr0));
    auto vload = [&](int db) __attribute__((always_inline)) {
      const i16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          reinterpret_cast<l_i16x4_t*>(static_cast<uintptr_t>(vr0 + 32 * db)));
      const i16x4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          reinterpret_cast<l_i16x4_t*>(static_cast<uintptr_t>(vr0 + 32 * db + 32 * kRow)));
      const u32x2_t w0 = __builtin_bit_cast(u32x2_t, v0), w1 = __builtin_bit_cast(u32x2_t, v1);
      return u32x4_t{w0[0], w0[1], w1[0], w1[1]};
    };
    constexpr int kVA = 3;  // value operands in flight
    u32x4_t vb[kVA + 1];
    sfor<kVA>([&](auto D) { vb[D] = vload(D); });
    sfor<kDB>([&](auto D) {
      constexpr int db = decltype(D)::value;
      if constexpr (db + kVA < kDB) vb[(db + kVA) % (kVA + 1)] = vload(db + kVA);
      // next tile's softmax in quarters, spread over the first output tiles
      if constexpr (kSoftmaxInPV && db % 4 == 1 && db / 4 < 2 * HB)
        softmax_part((db / 4) & 1, (db / 4) >> 1, pn);
#pragma unroll
      for (int hb = 0; hb < HB; hb++) o[hb][db] = mfma(p[hb], vb[db % (kVA + 1)], o[hb][db]);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // The running max starts at the first tile's max and is otherwise fixed:
  // probabilities up to 2^kTau are exact enough in fp32/bf16.  A score that
  // exceeds it by more than kTau makes the workgroup run the split again,
  // with m_est = the largest score of the whole first run, so the second
  // run never needs a third.  (The accumulators are never rescaled: a
  // rescale branch in the loop makes the compiler copy all of them on every
  // tile.)
  //
  // Pipeline (one barrier per tile): iteration i runs QK(i+1) with
  // dequant(i+2) interleaved, then P V(i) with softmax(i+1) interleaved;
  // three key tiles (PV, QK, dequant target) and two raw stages (the one
  // being dequantized and the one in flight).
  auto run = [&]() __attribute__((always_inline)) -> bool {
#pragma unroll
    for (int hb = 0; hb < HB; hb++) {
#pragma unroll
      for (int db = 0; db < kDB; db++) o[hb][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      m_run[hb] = m_est[hb];
      l_run[hb] = 0.f;
    }
    if (tid < (kSbRow + 12) / 4) reinterpret_cast<uint32_t*>(zero_sb)[tid] = 0u;
    issue(0, chunk_of(0));
    issue(1, chunk_of(1));
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerWave) : "memory");
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    dequant_all(0);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(2, chunk_of(2));
    const uint8_t* cnext = chunk_of(3);
    qk_dequant(0, 0);
    bool redo = softmax_check(0, 0);
    u32x4_t p[HB];
#pragma unroll
    for (int hb = 0; hb < HB; hb++)
#pragma unroll
      for (int tb = 0; tb < 2; tb++) softmax_part(tb, hb, p);

    for (int i = 0; i < ntiles; i++) {
      // raw(i+2) has landed and K(i+1) is complete in every wave; PV(i-1)
      // is done with kt[(i+2) % 3] and dequant(i+1) with raw[(i+1) % 2]
      asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      int ob = 0;
      asm volatile("" : "+v"(ob));
      issue(i + 3, cnext);
      cnext = chunk_of(i + 4);
      qk_dequant(i + 1, ob);
      redo |= softmax_check(i + 1, ob);
      u32x4_t pn[HB];
      if constexpr (!kSoftmaxInPV) {
#pragma unroll
        for (int hb = 0; hb < HB; hb++)
#pragma unroll
          for (int tb = 0; tb < 2; tb++) softmax_part(tb, hb, pn);
      }
      pv_softmax(i, ob, p, pn);
#pragma unroll
      for (int hb = 0; hb < HB; hb++) p[hb] = pn[hb];
    }
    // the extra tile ntiles was all masked: its probabilities are zero and
    // its sum is not added (l_run got zeros); every raw-tile load has landed
    // before the staging buffers are reused or the workgroup ends; then
    // agree on a second run
    if (lane == 0) restart_flag[wave] = redo ? 1 : 0;
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const u32x4_t f = *reinterpret_cast<const u32x4_t*>(&restart_flag[0]);
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
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    float ir[4];
#pragma unroll
    for (int e = 0; e < 4; e++) ir[e] = __shfl(inv, 4 * g + e);
    // whole sequence: the output; a split: its normalized partial (bf16)
    // and (max, sum)
    uint16_t* dst = a.n_splits == 1 ? a.out : a.ws_o;
    const int64_t dss = a.n_splits == 1 ? a.o_ss : static_cast<int64_t>(a.H) * kDV;
    const int64_t dsh = a.n_splits == 1 ? a.o_sh : kDV;
    const int64_t row = a.n_splits == 1 ? b : static_cast<int64_t>(slot);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int h = hw + 16 * hb + 4 * g + e;
      if (h < a.H) {
        uint16_t* op = dst + row * dss + static_cast<int64_t>(h) * dsh + n;
#pragma unroll
        for (int db = 0; db < kDB; db++) op[16 * db] = f32_to_bf16(o[hb][db][e] * ir[e]);
      }
    }
    const int h = hw + 16 * hb + n;
    if (a.n_splits > 1 && g == 0 && h < a.H) {
      a.ws_ml[(slot * a.H + h) * 2] = m_run[hb];
      a.ws_ml[(slot * a.H + h) * 2 + 1] = lt;
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
