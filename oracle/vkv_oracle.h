/*
 * vkv_oracle.h -- CPU restatement of the reference's KV-cache arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product library never links it.
 *
 * Every function names the reference file:line it restates.  Paths are
 * relative to the osaurus-ai/vmlx-swift checkout.
 *
 * dtype codes (same numbering as the product ABI): 0 = f32, 1 = f16, 2 = bf16.
 */
#ifndef VKV_ORACLE_H
#define VKV_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions (IEEE round-to-nearest-even) ---- */
uint16_t vkvo_f32_to_bf16(float f);
float vkvo_bf16_to_f32(uint16_t h);
uint16_t vkvo_f32_to_f16(float f);
float vkvo_f16_to_f32(uint16_t h);
void vkvo_to_f32(const void *src, int dtype, int64_t n, float *dst);
void vkvo_from_f32(const float *src, int64_t n, int dtype, void *dst);

/* ---- affine quantization (quantized.h:2393-2497, Metal semantics) ----
 * w: rows x D elements of `dtype`, contiguous.  wq: rows x (D*bits/32) u32,
 * little-endian packing, element i of a word at bit bits*i.  scales/biases:
 * rows x (D/group) of `dtype`.  Returns the number of exact .5 ties met by
 * round() (those are where a half-even rounding backend would differ). */
int64_t vkvo_quantize(const void *w, int dtype, int64_t rows, int D, int group,
                      int bits, uint32_t *wq, void *scales, void *biases);

/* Dequantize (quantized.h:2498-2560): out = scale * q + bias in T.
 * rule 0: the exact value rounded once to T (a fused multiply-add; the rule
 * this build's kernels use); rule 1: T(T(scale * q) + bias), two roundings.
 * The reference tree does not fix which one its compiled kernel performs. */
void vkvo_dequantize(const uint32_t *wq, const void *scales, const void *biases,
                     int dtype, int64_t rows, int D, int group, int bits, int rule,
                     void *out);
/* Number of elements where rules 0 and 1 above give different values. */
int64_t vkvo_dequantize_rule_split(const uint32_t *wq, const void *scales,
                                   const void *biases, int dtype, int64_t rows, int D,
                                   int group, int bits);

/* ---- float decode SDPA (MLXFast.swift:173-218, sdpa_vector.h:15-177) ----
 * q [B,Hq,L,D], k [B,Hkv,T,D], v [B,Hkv,T,Dv] as f32 values (exact images of
 * the stored dtype); q is scaled in f32 (sdpa_vector.h:78).  Accumulation is
 * f64.  mask_mode: 0 none, 1 causal (key i visible to query row l when
 * i <= T - L + l), 2 bool, 3 additive.  Mask element (b,h,l,t) lives at
 * mask[b*msb + h*msh + l*msl + t*mst].  An additive mask is rounded to the
 * query dtype q_dtype and keys below its lowest finite value are skipped
 * (sdpa_vector.h:15-38, :105-121); masked keys are skipped; a row with no
 * visible key (and no sink) returns zeros (sdpa_vector.h:160-166).  sinks
 * (NULL = none): [Hq] logits, one extra softmax term per query head with a
 * zero value row (:93-96).  out [B,Hq,L,Dv] f64. */
void vkvo_sdpa(const float *q, const float *k, const float *v, int B, int Hq,
               int Hkv, int L, int T, int D, int Dv, float scale, int mask_mode,
               const uint8_t *bmask, const float *fmask, int64_t msb, int64_t msh,
               int64_t msl, int64_t mst, int q_dtype, const float *sinks, double *out);

/* ---- quantized SDPA (KVCache.swift:1909-1997) ----
 * q [B,Hq,L,D] f32 values of dtype q_dtype; the queries are first scaled in
 * the input dtype: qs = T(q * T(scale)) (MLXArray+Ops.swift:235-237,
 * DType.swift:389-396).  Keys/values in the reference layout
 * [B,Hkv,T,D*bits/32] u32 with scales/biases [B,Hkv,T,D/group] given as f32
 * values of the stored dtype.  Masks as in vkvo_sdpa except that masked
 * scores are filled with finfo(T).min before the softmax (so a fully masked
 * row averages V, KVCache.swift:1950-1975).
 * rounding selects the arithmetic:
 *   0  exact: scores, softmax and P.V in f64 (the limit of every rounding);
 *   1  the reference's rounding on the vector path (affine_qmv / qvm,
 *      quantized.h:1493-1764): scores accumulated exactly from the exact
 *      dequantized keys, then stored in T (quantizedMM returns the query
 *      dtype, KVCache.swift:1945-1949); an f32 additive mask promotes them
 *      to f32 (:1969); softmax (:1982) with fp32 internals (the arithmetic
 *      of precise: true) and its weights stored in T; P.V accumulated
 *      exactly over the T weights;
 *   2  as 1 on the matrix path (affine_qmm, quantized.h:568-576, :686-713):
 *      keys and values are first dequantized to T (rule 0 above);
 *   3  as 1 with the softmax's internal arithmetic in T: the kernels'
 *      default AccT = T (softmax.h:10, :100), which softmax(precise: false)
 *      selects for f16/bf16 -- the reference's decode arithmetic; rows of
 *      up to 4096 keys reduce as softmax_single_row, longer rows as
 *      softmax_looped (see softmax_row in vkv_oracle.c);
 *   4  as 3 on the matrix path: the reference's multi-token arithmetic.
 * wbound (optional, [B,Hq,L,D], rounding modes only): the most the
 * reference's roundings can move each output away from the exact softmax of
 * the rounded scores: sum_t |w_t - pe_t| |v_t| for the weights stored in T,
 * plus, for each score within 2^-17 sum_d |q_d k_td| of a T rounding
 * boundary (where any fp32 accumulation may land on either side), the exact
 * output change of rounding it the other way.  fbound (optional, same
 * shape): the score-boundary term alone, for a kernel that reproduces the
 * reference's weights from the same stored scores: for each such score,
 * the move of the output when it is stored the other way, computed in the
 * mode's own arithmetic (the rounded softmax can move its normaliser, and
 * with it every weight); the flips of a row are added. */
void vkvo_quantized_sdpa(const float *q, int q_dtype, const uint32_t *kq,
                         const float *ks, const float *kb, const uint32_t *vq,
                         const float *vs, const float *vb, int B, int Hq, int Hkv,
                         int L, int T, int D, int group, int bits, float scale,
                         int mask_mode, const uint8_t *bmask, const float *fmask,
                         int64_t msb, int64_t msh, int64_t msl, int64_t mst,
                         int rounding, double *out, double *wbound, double *fbound);

/* ---- MLA absorbed-latent decode (GLM4MOELite.swift:233-290,
 * AttentionUtils.swift:43-75) ----
 * One shared latent head.  q [B,H,Dk] f32 values (Dk = 576 = 512 latent + 64
 * rope).  The cache holds Dk-dim entries quantized affine (bits, group) in
 * the reference layout [B,T,Dk*bits/32] u32 + scales/biases [B,T,Dk/group]
 * (f32 values of the stored dtype).  Keys are the dequantized entries (exact,
 * f64), values their first Dv dims.  lens[b] valid tokens for batch row b.
 * out [B,H,Dv] f64. */
void vkvo_mla_decode(const float *q, const uint32_t *cq, const float *cs,
                     const float *cb, int B, int H, int T, const int32_t *lens,
                     int Dk, int Dv, int group, int bits, float scale, double *out);

/* CPU-baseline entry: the same quantized decode as vkvo_quantized_sdpa (with
 * its rounding modes) for L == 1 without a mask, over `nseq` independent sequences of lengths lens[],
 * each stored contiguously [Hkv,T_i,...] at the given element offsets.  Uses
 * up to `threads` OpenMP threads (1 = scalar). */
void vkvo_quantized_decode_batch(const float *q, int q_dtype, const uint32_t *kq,
                                 const float *ks, const float *kb, const uint32_t *vq,
                                 const float *vs, const float *vb, int nseq,
                                 const int32_t *lens, const int64_t *tok_off, int Hq,
                                 int Hkv, int D, int group, int bits, float scale,
                                 int rounding, int threads, double *out);

#ifdef __cplusplus
}
#endif
#endif
