// vkv_kvread.h -- device-side reads of one K or V element (float blocks,
// the paged affine chunk format, or reference-layout affine tuples), shared
// by the generic attention kernels (vkv_kernels.hip) and the
// reference-arithmetic attention (vkv_refattn.hip).
#pragma once

#include "vkv_device.h"
#include "vkv_internal.h"

namespace vkv {

// ---------------------------------------------------------------- KV access

struct TokLoc {
  int64_t blk;  // block id (paged) or sequence index (dense)
  int64_t tib;  // token index inside the block (or sequence)
};

__device__ __forceinline__ TokLoc locate(const KVSrc& kv, int64_t s, int64_t t) {
  TokLoc r;
  if (kv.table) {
    r.blk = kv.table[s * kv.table_stride + t / kv.block_size];
    r.tib = t % kv.block_size;
  } else {
    r.blk = s;
    r.tib = t;
  }
  return r;
}

__device__ __forceinline__ const uint8_t* at(const Comp& c, const TokLoc& l, int64_t h) {
  return c.ptr + l.blk * c.sb + h * c.sh + l.tib * c.st;
}

// code of element d of a token-major codes row
template <int BITS>
__device__ __forceinline__ uint32_t code_tm(const uint8_t* row, int d) {
  if constexpr (BITS == 8) return row[d];
  return (row[d >> 1] >> (4 * (d & 1))) & 15u;
}

// Raw affine code of element d of the token at `l` (which: 0 = K, 1 = V)
// with its stored scale and bias, for either the paged chunk format or the
// reference layout.  Values of a keys-only (MLA) chunk are its key entries.
template <int DT, int BITS>
__device__ __forceinline__ uint32_t qcode(const KVSrc& kv, const TokLoc& l, int64_t h, int d,
                                          int which, int group, float* s, float* b) {
  using E = Elem<DT>;
  const int g = d / group;
  if (kv.qfmt) {
    const uint8_t* chunk = kv.base + l.blk * kv.block_bytes + h * kv.head_bytes;
    const typename E::T* sb = reinterpret_cast<const typename E::T*>(chunk + kv.sb_off);
    const bool ko = kv.keys_only != 0;
    const int w = (which && !ko) ? 1 : 0;
    *s = E::load(sb + qsb_index(l.tib, w, g, 0, kv.G, ko));
    *b = E::load(sb + qsb_index(l.tib, w, g, 1, kv.G, ko));
    if (w == 0) {
      constexpr int per = 32 / BITS;
      const uint32_t word = *reinterpret_cast<const uint32_t*>(
          chunk + kv.kc_off + qk_word_off(l.tib, d / per, kv.D, BITS));
      return (word >> (BITS * (d % per))) & ((1u << BITS) - 1u);
    }
    int sh;
    const uint32_t word =
        *reinterpret_cast<const uint32_t*>(chunk + kv.vc_off + qv_word_off(l.tib, d, kv.D, BITS, &sh));
    return (word >> sh) & ((1u << BITS) - 1u);
  }
  const Comp& cc = which ? kv.vc : kv.kc;
  const Comp& sc = which ? kv.vs : kv.ks;
  const Comp& bc = which ? kv.vb : kv.kb;
  *s = E::load(reinterpret_cast<const typename E::T*>(at(sc, l, h)) + g);
  *b = E::load(reinterpret_cast<const typename E::T*>(at(bc, l, h)) + g);
  return code_tm<BITS>(at(cc, l, h), d);
}

// K (which 0) or V (which 1) element as float: float blocks load it,
// affine blocks dequantize it as fp32 scale * code + bias.
template <int DT, int BITS>
__device__ __forceinline__ float kv_at(const KVSrc& kv, const TokLoc& l, int64_t h, int d, int which,
                                       int group) {
  using E = Elem<DT>;
  if constexpr (BITS == 0) {
    const Comp& c = which ? kv.vc : kv.kc;
    return E::load(reinterpret_cast<const typename E::T*>(at(c, l, h)) + d);
  } else {
    float s, b;
    const uint32_t c = qcode<DT, BITS>(kv, l, h, d, which, group, &s, &b);
    return fmaf(s, static_cast<float>(c), b);
  }
}

}  // namespace vkv
