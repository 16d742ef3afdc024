/*
 * vkv.h -- C ABI of the MI355X KV-cache engine (libvkv.so).
 *
 * This is the drop-in boundary for the KV-cache hot path of vmlx-swift.  The
 * reference reaches its tensor arithmetic through mlx-c (the headers under
 * `Source/Cmlx/include/mlx/c/`, exposed to Swift by `Source/Cmlx/include/module.modulemap:1-3`)
 * and its cache state machines through the Swift `KVCache` protocol
 * (`Libraries/MLXLMCommon/KVCache.swift:38-77`).  Each entry point below
 * names the reference interface it replaces.  Paths are relative to the
 * osaurus-ai/vmlx-swift checkout.
 *
 * Conventions (mirroring mlx-c, `Libraries/CmlxDistributedShim/
 * MlxCDistributed.cpp:11-28`):
 *   - every call returns int: 0 = success, non-zero = failure; nothing throws
 *     across the ABI.  vkv_last_error() gives the message of the calling
 *     thread's last failure.
 *   - device memory behind a cache / pool handle is owned by the handle.
 *     Arrays and views returned by a call stay valid until the next mutating
 *     call on the same handle (the reference returns MLX views with the same
 *     lifetime, KVCache.swift:465-508).
 *   - every call that launches work takes a hipStream_t passed as void*
 *     (NULL = the default stream); work is stream-ordered, calls do not
 *     synchronize unless they say so.
 *   - cache handles are single-writer (the reference's caches take no
 *     locks); the prefix-cache manager is internally locked like
 *     PagedCacheManager (PagedCacheManager.swift:51-52).
 */
#ifndef VKV_H
#define VKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VKV_ABI_VERSION 2

/* ------------------------------------------------------------------ types */

/* element types (the subset of mlx_dtype the cache path uses) */
enum {
  VKV_F32 = 0,
  VKV_F16 = 1,
  VKV_BF16 = 2,
  VKV_U32 = 3,
  VKV_I32 = 4,
  VKV_U8 = 5,
  VKV_BOOL = 6
};

/* A strided device array of up to 4 dims (strides in elements).  Replaces
 * mlx_array at this boundary (`Source/Cmlx/include/mlx/c/array.h`). */
typedef struct vkv_array {
  void *data;
  int32_t dtype;
  int32_t ndim;
  int64_t shape[4];
  int64_t strides[4];
} vkv_array;

/* Paged KV storage as the attention kernels read it.  Produced by
 * vkv_pool_view() and vkv_cache_update_quantized(); it has no reference
 * counterpart (the reference concatenates blocks back into one array,
 * Cache/CacheHelpers.swift:431-552).
 *
 * Block format of one (layer, block, kv head) chunk, head_bytes long:
 *   float blocks (bits == 0):  K [block_size][head_dim] dtype,
 *                              V [block_size][head_dim] dtype
 *   affine blocks (bits 4/8):  K codes [block_size][head_dim*bits/8] bytes,
 *                              V codes [head_dim][block_size*bits/8] bytes
 *                                (dim-major: the tokens of one dim are
 *                                contiguous, which is the operand order the
 *                                P.V contraction needs),
 *                              K scales, K biases, V scales, V biases
 *                                [block_size][head_dim/group] dtype each.
 *   keys-only (flags & VKV_VIEW_KEYS_ONLY, MLA latent): K codes, K scales,
 *                                K biases only; values are the first
 *                                v_head_dim dims of the key entry.
 * Codes pack element i of a 32-bit little-endian word at bit bits*i, the
 * reference's packing (quantized.h:2455-2497). */
enum { VKV_VIEW_KEYS_ONLY = 1 };

typedef struct vkv_paged_view {
  const void *base;            /* device address of block 0 of this layer */
  int32_t dtype;               /* element dtype (float) / scale-bias dtype */
  int32_t bits;                /* 0, 4 or 8 */
  int32_t group_size;          /* affine group size (64) */
  int32_t n_kv_heads;
  int32_t head_dim;            /* key dims */
  int32_t v_head_dim;          /* value dims (== head_dim unless keys-only) */
  int32_t block_size;          /* tokens per block */
  int32_t flags;
  int64_t block_bytes;         /* bytes of one block (all kv heads) */
  int64_t head_bytes;          /* bytes of one (block, kv head) chunk */
  const int32_t *block_table;  /* device [n_seqs, table_stride] block ids */
  int32_t table_stride;
  const int32_t *seq_lens;     /* device [n_seqs] valid tokens per sequence;
                                  NULL = every sequence holds max_len */
  int32_t n_seqs;
  int32_t max_len;             /* host-side upper bound of seq_lens */
} vkv_paged_view;

typedef struct vkv_cache_s *vkv_cache;
typedef struct vkv_pool_s *vkv_pool;
typedef struct vkv_prefix_s *vkv_prefix;

/* ------------------------------------------------------------------ errors */

/* Last error message of the calling thread ("" when none).  Replaces
 * mlx_set_error_handler's message delivery (mlx/c/error.h:15-24). */
const char *vkv_last_error(void);
int vkv_abi_version(void);
/* Count of HIP devices visible to the library (0 on a host without a GPU). */
int vkv_device_count(int32_t *count);

/* ------------------------------------------------ quantization operators */

/* mlx_quantize (mlx/c/ops.h:801-808) -> affine_quantize
 * (mlx-generated/metal/quantized.h:2393-2497), affine mode only.
 * w: [..., D] f16/bf16/f32, last dim contiguous, D % group_size == 0.
 * Writes wq [..., D*bits/32] u32, scales/biases [..., D/group_size] of w's
 * dtype (all contiguous, caller-allocated).  bits in {4, 8}. */
int vkv_quantize_affine(const vkv_array *w, int32_t group_size, int32_t bits,
                        vkv_array *wq, vkv_array *scales, vkv_array *biases,
                        void *stream);

/* mlx_dequantize (mlx/c/ops.h:359-369) -> affine_dequantize
 * (quantized.h:2498-2560): out = scale * q + bias, one fp32 fused
 * multiply-add rounded once to the output dtype (scales' dtype). */
int vkv_dequantize_affine(const vkv_array *wq, const vkv_array *scales,
                          const vkv_array *biases, int32_t group_size, int32_t bits,
                          vkv_array *out, void *stream);

/* ----------------------------------------------------------- attention */

enum { VKV_MASK_NONE = 0, VKV_MASK_CAUSAL = 1, VKV_MASK_ARRAY = 2 };

/* mlx_fast_scaled_dot_product_attention (mlx/c/fast.h:189-198) as called
 * by MLXFast.scaledDotProductAttention (MLX/MLXFast.swift:203-218):
 * q [B,Hq,L,D], k [B,Hkv,T,D], v [B,Hkv,T,Dv] (strided, same float dtype),
 * Hq % Hkv == 0 (GQA without tiling).  fp32 softmax and accumulation.
 * mask_mode VKV_MASK_ARRAY takes a bool mask, or an additive mask in f32 or
 * q's dtype, broadcastable to [B,Hq,L,T] (stride 0 on broadcast dims); an
 * additive mask is read as q's dtype and keys whose mask is below that
 * dtype's lowest finite value are skipped (sdpa_vector.h:15-38, :105-121).
 * sinks (NULL = none): [Hq] logits (f32 or a 16-bit float, read as q's
 * dtype), one per query head, each an extra softmax term with a zero value
 * row (sdpa_vector.h:93-96, :257-260).  out [B,Hq,L,Dv] in q's dtype.  A
 * row with no visible key yields zeros. */
int vkv_sdpa(const vkv_array *q, const vkv_array *k, const vkv_array *v, float scale,
             int32_t mask_mode, const vkv_array *mask, const vkv_array *sinks,
             vkv_array *out, void *stream);

/* quantizedScaledDotProductAttention (MLXLMCommon/KVCache.swift:1909-1997)
 * over quantized tuples in the reference layout: k_wq [B,Hkv,T,D*bits/32]
 * u32, k_scales/k_biases [B,Hkv,T,D/group] (likewise v_*).  Queries are
 * scaled in their own dtype first (T(q * T(scale))), masked scores are
 * filled with the dtype's lowest value before the softmax, so a fully masked
 * row averages V (unlike vkv_sdpa). */
int vkv_quantized_sdpa(const vkv_array *q, const vkv_array *k_wq,
                       const vkv_array *k_scales, const vkv_array *k_biases,
                       const vkv_array *v_wq, const vkv_array *v_scales,
                       const vkv_array *v_biases, int32_t group_size, int32_t bits,
                       float scale, int32_t mask_mode, const vkv_array *mask,
                       vkv_array *out, void *stream);

/* Decode attention over paged KV: one query token per sequence.
 * q [n_seqs, Hq, D] (strided), out [n_seqs, Hq, Dv] in q's dtype.  For
 * affine views the arithmetic is the reference's quantized SDPA
 * (KVCache.swift:1909-1997, queries scaled in their dtype); for float views
 * it is MLXFast SDPA (sdpa_vector.h:15-177).  Sequence s attends to its
 * seq_lens[s] tokens; a sequence of length 0 yields zeros.  Replaces the
 * reference's pad-and-concatenate batching (BatchEngine/BatchKVCache.swift:
 * 83-113, 177-193) for the continuous-batching decode step. */
int vkv_paged_sdpa(const vkv_array *q, const vkv_paged_view *kv, float scale,
                   vkv_array *out, void *stream);

/* vkv_paged_sdpa without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops or harnesses that forbid
 * hipMalloc).  Same arguments, arithmetic and results as vkv_paged_sdpa;
 * the split-K partials go to a fixed 64 MiB device array that the library
 * holds on each GPU it runs on until the process ends, instead of the
 * per-stream workspace.  A call whose partials do not fit (about 1000
 * (sequence, kv head) pairs at head_dim 128 on the matrix-core path) fails
 * with an error naming the size.  Calls share the array of their device:
 * calls that overlap on one device (two streams, two threads) race. */
int vkv_paged_sdpa_noalloc(const vkv_array *q, const vkv_paged_view *kv, float scale,
                           vkv_array *out, void *stream);

/* Absorbed-latent MLA decode (MLXLLM/Models/GLM4MOELite.swift:233-290 via
 * MLXLMCommon/AttentionUtils.swift:43-75): one shared latent head; kv is a
 * keys-only affine view (entries of head_dim = 576 dims, values = first
 * v_head_dim = 512 dims).  q [n_seqs, H, head_dim] bf16, out [n_seqs, H,
 * v_head_dim] bf16.  QK^T and PV run as bf16/f16 MFMA contractions over the
 * H query heads. */
int vkv_mla_decode(const vkv_array *q, const vkv_paged_view *kv, float scale,
                   vkv_array *out, void *stream);

/* quantizedScaledDotProductAttention(queries:quantizedKeys:quantizedValues:
 * scale:mask:groupSize:bits:) (KVCache.swift:1909-1997) over the paged view
 * that vkv_cache_update_quantized returns (or a pool view of affine
 * blocks), for any number of query tokens: the binding for a model that
 * calls updateQuantized and then quantizedScaledDotProductAttention itself
 * (GPTOSS.swift:239-248, MiMoV2Flash.swift:36-45) without materializing the
 * tuples.  q [n_seqs,Hq,L,D], out [n_seqs,Hq,L,Dv] in the view's dtype;
 * masks as in vkv_quantized_sdpa (causal: query l of a sequence of length
 * T sees keys t <= T - L + l).  Same arithmetic as vkv_quantized_sdpa. */
int vkv_quantized_paged_sdpa(const vkv_array *q, const vkv_paged_view *kv, float scale,
                             int32_t mask_mode, const vkv_array *mask, vkv_array *out,
                             void *stream);

/* attentionWithCacheUpdate(queries:keys:values:cache:scale:mask:)
 * (AttentionUtils.swift:77-143), one call: with cache == NULL, SDPA over
 * keys/values; with a QuantizedKVCache, updateQuantized then quantized SDPA
 * over the whole cache (the matrix-core decode kernel for one query token
 * without a mask, which then also quantizes the new token into the cache
 * itself, in the same launch and with the same bits, where the cache has
 * group 64 and at most 8 query heads a kv head); with any other cache, update then SDPA over the returned
 * keys/values, where a VKV_MASK_NONE mask is replaced by the cache's own
 * array mask if makeMask(n:windowSize:nil:returnArray:true) gives one
 * (called after the update, as the reference does).  q [B,Hq,L,D],
 * keys/values [B,Hkv,L,D] (the new tokens), out [B,Hq,L,Dv].  sinks as in
 * vkv_sdpa, for the float caches only (a quantized cache refuses them, as
 * the models that pass sinks do, Libraries/MLXLLM/Models/GPTOSS.swift:
 * 223-235). */
int vkv_attention_with_cache_update(const vkv_array *q, const vkv_array *keys,
                                    const vkv_array *values, vkv_cache cache, float scale,
                                    int32_t mask_mode, const vkv_array *mask,
                                    const vkv_array *sinks, vkv_array *out, void *stream);

/* ------------------------------------------------------- per-layer caches */

enum {
  VKV_CACHE_SIMPLE = 0,    /* KVCacheSimple    KVCache.swift:452-596 */
  VKV_CACHE_ROTATING = 1,  /* RotatingKVCache  KVCache.swift:605-958 */
  VKV_CACHE_QUANTIZED = 2, /* QuantizedKVCache KVCache.swift:961-1221 */
  /* CompilableKVCache (CompilableKVCache.swift:40-262): fixed [B,H,max,D]
   * buffers, max = params.max_size (default 4096), write offset in device
   * memory; update returns the whole buffers and makeMask always an array
   * mask [n, max] built on the device. */
  VKV_CACHE_COMPILABLE = 3,
  /* CompilableRotatingKVCache (BatchEngine/CompilableRotatingKVCache.swift:
   * 1-265): a RotatingKVCache whose buffers are allocated at maxSize once and
   * whose ring index and offset live in device memory. */
  VKV_CACHE_COMPILABLE_ROTATING = 4,
  /* TurboQuantKVCache (TurboQuant/TurboQuantKVCache.swift:70-671): float
   * KV while filling, then a TurboQuant-encoded prefix decoded once into a
   * float buffer followed by a float window.  vkv_cache_create gives the
   * reference's defaults (keyBits 3, valueBits 3, 4 sink tokens, 64
   * residual tokens; params.bits > 0 sets both bit widths). */
  VKV_CACHE_TURBOQUANT = 5,
  /* CompilableTurboQuantKVCache (BatchEngine/CompilableTurboQuantKVCache.swift:
   * 57-294): a compressed TurboQuantKVCache whose window writes go to the
   * offset held in device memory (update returns the whole unified buffers,
   * makeMask an array mask over them); made by vkv_turboquant_to_compilable. */
  VKV_CACHE_COMPILABLE_TURBOQUANT = 6
};

typedef struct vkv_cache_params {
  int32_t kind;
  int32_t step;        /* growth step, default 256 (KVCache.swift:455, :966) */
  int32_t max_size;    /* rotating window (RotatingKVCache.init maxSize);
                          CompilableKVCache maxLength (default 4096) */
  int32_t keep;        /* rotating keep prefix */
  int32_t group_size;  /* quantized: 64 */
  int32_t bits;        /* quantized: 4 or 8 (default 8, KVCache.swift:970) */
} vkv_cache_params;

/* Cache construction: KVCacheSimple(), RotatingKVCache(maxSize:keep:step:),
 * QuantizedKVCache(groupSize:bits:).  Zero fields take the reference
 * defaults (step 256, group 64, bits 8, keep 0). */
int vkv_cache_create(const vkv_cache_params *params, vkv_cache *out);
int vkv_cache_destroy(vkv_cache cache);
/* copy() (KVCache.swift:583-591, :947-954, :1188-1195): deep, independent. */
int vkv_cache_copy(vkv_cache cache, void *stream, vkv_cache *out);

/* update(keys:values:) (KVCache.swift:465-508, :791-799).  keys [B,Hkv,S,D],
 * values [B,Hkv,S,Dv] (strided).  out_keys/out_values receive views of the
 * cached K/V exactly as the reference returns them (trimmed to offset, or the
 * whole ring once a rotating cache has wrapped).  Fails on a quantized cache
 * like the reference traps (KVCache.swift:1126-1130). */
int vkv_cache_update(vkv_cache cache, const vkv_array *keys, const vkv_array *values,
                     void *stream, vkv_array *out_keys, vkv_array *out_values);

/* updateQuantized(keys:values:) (KVCache.swift:1049-1122): quantizes the new
 * tokens (affine, bit-exact with quantized.h:2393-2497) into the cache and
 * returns the whole cache as a paged view: the updated tuples in the paged
 * block format, which vkv_quantized_paged_sdpa (any query length, masks)
 * and vkv_paged_sdpa (one decode token) attend over directly.  The
 * reference-layout tuples themselves come from
 * vkv_cache_update_quantized_tuples (below). */
int vkv_cache_update_quantized(vkv_cache cache, const vkv_array *keys,
                               const vkv_array *values, void *stream,
                               vkv_paged_view *out);

/* updateQuantized(keys:values:) (KVCache.swift:1049-1122) with the
 * reference's return value: out[6] receives the keys' (wq, scales, biases)
 * then the values', each [B, Hkv, offset, *] in the reference layout
 * (wq u32 [.., D * bits / 32], scales and biases in the K/V dtype [..,
 * D / group]), views of cache-owned arrays whose dim(2) is the cache's
 * capacity (the reference's keys.0.dim(2)).  The cache keeps them beside
 * its paged store and brings them up to date from it for the tokens
 * written since the previous call (a trim or a state setter included), so
 * a decode step costs its new tokens, not the whole cache; when the
 * capacity grows they are re-created and gathered whole, as the
 * reference's arrays are.  The views stay valid until the next call that
 * grows the cache.  The paged view (vkv_cache_update_quantized) is the
 * same cache: both may be used on one cache. */
int vkv_cache_update_quantized_tuples(vkv_cache cache, const vkv_array *keys,
                                      const vkv_array *values, void *stream, vkv_array *out);

/* The cache's class (VKV_CACHE_*): the dynamic type the reference's
 * savePromptCache switches on (KVCache.swift:1627-1646). */
int vkv_cache_kind(vkv_cache cache, int32_t *kind);

/* offset / maxSize / isTrimmable / trim(n) (KVCache.swift:38-77). */
int vkv_cache_offset(vkv_cache cache, int64_t *offset);
/* offset setter (BaseKVCache.offset, KVCache.swift:256-262; the device
 * counter of the fixed-buffer caches, CompilableKVCache.swift:96-104). */
int vkv_cache_set_offset(vkv_cache cache, int64_t offset);
int vkv_cache_max_size(vkv_cache cache, int64_t *max_size); /* -1 = none */
int vkv_cache_is_trimmable(vkv_cache cache, int32_t *trimmable);
int vkv_cache_trim(vkv_cache cache, int64_t n, int64_t *trimmed);
/* Physical token capacity (the reference's keys.dim(2)); no protocol
 * counterpart, exposed so growth can be checked against the reference. */
int vkv_cache_capacity(vkv_cache cache, int64_t *capacity);

/* state getter (KVCache.swift:527-547, :801-823, :1133-1166): fills
 * `arrays` (room for 6) and *count: 2 for float caches (views), 6 for the
 * quantized cache (keys wq/scales/biases, values wq/scales/biases in the
 * reference layout, materialized into cache-owned memory). */
int vkv_cache_state(vkv_cache cache, void *stream, vkv_array *arrays, int32_t *count);
/* state setter: copies the arrays in (2 or 6, reference layout).  For
 * KVCacheSimple the offset becomes dim(2); for the rotating and quantized
 * caches offset comes from metaState, as in the reference. */
int vkv_cache_set_state(vkv_cache cache, const vkv_array *arrays, int32_t count,
                        void *stream);
/* metaState (KVCache.swift:824-853, :1168-1177): NUL-separated strings in
 * buf; *count receives the number of strings. */
int vkv_cache_meta_state(vkv_cache cache, char *buf, int64_t buf_len, int32_t *count);
int vkv_cache_set_meta_state(vkv_cache cache, const char *const *strings, int32_t count);

/* makeMask(n:windowSize:returnArray:) (KVCache.swift:287-311, :890-927).
 * window <= 0 means nil.  *mode receives VKV_MASK_*; for VKV_MASK_ARRAY,
 * *mask receives a bool array owned by the cache ([n, offset+n] or the
 * rolled [maskSize] row of the rotating single-token case). */
int vkv_cache_make_mask(vkv_cache cache, int32_t n, int32_t window, int32_t return_array,
                        void *stream, int32_t *mode, vkv_array *mask);

/* ---- TurboQuant KV codec (Libraries/MLXLMCommon/TurboQuant/) ----
 * EncodedKeys / EncodedValues (TQEncodedData.swift:38-170) as device
 * arrays, in the layouts TQDiskSerializer writes: codes of index_bits each
 * and QJL signs packed flat into u32 words (TQBitPack.swift: value e of the
 * [B, H, Tc, D] tensor in word e / (32 / bits) at bit (e % (32 / bits)) *
 * bits), f16 norms [B, H, Tc, 1], and the exact sink / tail tokens
 * [B, H, n, D] in the input dtype (ndim 0 when absent).  Values have no
 * qjl / res_norms (ndim 0). */
typedef struct vkv_tq_encoded {
  vkv_array indices;
  vkv_array qjl;
  vkv_array res_norms;
  vkv_array vec_norms;
  vkv_array sink;
  vkv_array tail;
  int32_t shape[4];    /* the compressed [B, H, Tc, D] */
  int32_t index_bits;  /* keys: keyBits - 1 (at least 1); values: valueBits */
  int32_t seed;        /* EncoderState seed (42) */
} vkv_tq_encoded;

typedef struct vkv_tq_info {
  int32_t phase;          /* TQPhase: 0 fill, 1 compressed */
  int32_t has_encoded;    /* compressedKeys / compressedValues are present */
  int64_t prefix_tokens;  /* prefixTokenCount */
  int64_t window_tokens;  /* windowOffset */
  int32_t key_bits, value_bits, sink_tokens, residual_tokens;
} vkv_tq_info;

/* TurboQuantKVCache(keyBits:valueBits:sinkTokens:residualTokens:)
 * (TurboQuantKVCache.swift:139-150).  keyBits in [1, 9] (codes of
 * max(keyBits - 1, 1) bits plus one QJL bit), valueBits in [1, 8]. */
int vkv_turboquant_create(int32_t key_bits, int32_t value_bits, int32_t sink_tokens,
                          int32_t residual_tokens, vkv_cache *out);
/* TurboQuantKVCache.fromSimpleCache(_:keyBits:valueBits:sinkTokens:
 * residualTokens:) (:326-356): encodes the simple cache's K/V (sink tokens
 * and the last residual tokens kept exact), decodes them once into the
 * unified buffer and returns a compressed-phase cache at the source's
 * offset; an empty fill-phase cache when the source has no compressible
 * middle of at least 8 tokens. */
int vkv_turboquant_from_simple(vkv_cache simple, int32_t key_bits, int32_t value_bits,
                               int32_t sink_tokens, int32_t residual_tokens, void *stream,
                               vkv_cache *out);
/* TurboQuantKVCache.hasCompressibleMiddle (:152-162). */
int vkv_turboquant_has_compressible_middle(int64_t token_count, int32_t sink_tokens,
                                           int32_t residual_tokens, int32_t minimum,
                                           int32_t *out);
int vkv_turboquant_info(vkv_cache cache, vkv_tq_info *info);
/* compressedKeys / compressedValues (:94-95) as views owned by the cache;
 * fails when the cache holds none (fill phase, or restored from decoded
 * K/V). */
int vkv_turboquant_encoded(vkv_cache cache, vkv_tq_encoded *keys, vkv_tq_encoded *values);
/* serializedWindowState (:254-263): the exact tokens appended after the
 * compression, *present = 0 when there are none. */
int vkv_turboquant_window(vkv_cache cache, vkv_array *keys, vkv_array *values, int32_t *present);
/* restoreCompressed(encodedKeys:encodedValues:sourceOffset:windowKeys:
 * windowValues:) (:180-252): copies the records, decodes them with
 * EncoderState(dim, index_bits + 1 | index_bits, seed), then appends the
 * window, which must hold exactly sourceOffset - (encoded tokens) tokens
 * (NULL when none); a mismatch leaves the cache empty (offset 0), as in
 * the reference. */
int vkv_turboquant_restore_compressed(vkv_cache cache, const vkv_tq_encoded *keys,
                                      const vkv_tq_encoded *values, int64_t source_offset,
                                      const vkv_array *window_keys, const vkv_array *window_values,
                                      void *stream);
/* restoreFromDecodedKV(keys:values:sourceOffset:) (:281-322). */
int vkv_turboquant_restore_decoded(vkv_cache cache, const vkv_array *keys, const vkv_array *values,
                                   int64_t source_offset, void *stream);
/* A TurboQuant cache as pool pages, so that a compressed sequence joins a
 * paged batched decode (vkv_paged_sdpa over the pool) beside float or
 * affine sequences.  Under batching the reference compresses each slot's
 * cache (BatchEngine/BatchQuantize.swift:115-125 -> maybeQuantizeKVCache)
 * and BatchKVCache attends the plain K/V its update returns
 * (TurboQuantKVCache.swift:428-500: the decoded prefix, then the exact
 * window).  This writes tokens [first_token, first_token + n_tokens) of
 * those K/V, every batch row, into pool slots: slot_mapping is device int32
 * [B * n_tokens], row b's tokens at b * n_tokens (slot = block * block_size
 * + position, -1 skips a token).  Rows are cast to the pool dtype (round to
 * nearest even; an f32 pool holds them exactly) and quantized as any append
 * when the pool is affine.  After the compression write [0, offset); after
 * each later update write its new tokens (they sit in the window, exact). */
int vkv_turboquant_write_pool(vkv_cache cache, vkv_pool pool, int32_t layer,
                              const int32_t *slot_mapping, int64_t first_token, int64_t n_tokens,
                              void *stream);
/* The codec's host tables (EncoderState, TQEncoder.swift:88-107): the
 * rotation signs of (dim, seed) (TQHadamard.generateRandomSigns), the
 * Lloyd-Max codebook of (dim, bits) (TQCodebook.computeCodebook, 2^bits
 * floats) and the QJL matrix [dim, dim] (TQQJL.generateProjection with
 * seed + 1000).  Any output may be NULL.  Host only. */
int vkv_tq_tables(int32_t dim, int32_t bits, int32_t seed, float *signs, float *codebook,
                  float *qjl);

/* createBatchCausalMask(queryLen:offsets:effectiveKeyLens:windowSize:)
 * (BatchEngine/BatchMask.swift:44-115): the bool mask [batch, 1, n,
 * max_total] of a batched step in which slot b held offsets[b] tokens
 * before the step.  key_lens (NULL: offsets[b] + n) are the keys each
 * slot's update returns; a slot whose key length is below offsets[b] + n
 * has wrapped its ring and sees every key below its length.  window < 0
 * means no window (windowSize nil); window >= 0 also requires key j >=
 * query position - (window - 1).  *max_total receives the last dimension
 * (the largest key length).  With out == NULL nothing is launched (a size
 * query); otherwise out is a caller-owned, 16-byte aligned device buffer
 * of out_bytes >= batch * n * max_total.  The per-slot values are read on
 * the host and travel as kernel arguments (no allocation, no copy). */
int vkv_batch_causal_mask(int32_t n, const int32_t *offsets, const int32_t *key_lens,
                          int32_t batch, int32_t window, void *out, int64_t out_bytes,
                          void *stream, int32_t *max_total);

/* KVCacheSimple.toQuantized (KVCache.swift:561-581) and
 * QuantizedKVCache.toUnquantized (:1199-1220); new handles. */
int vkv_cache_to_quantized(vkv_cache simple, int32_t group_size, int32_t bits,
                           void *stream, vkv_cache *out);
int vkv_cache_to_unquantized(vkv_cache quantized, void *stream, vkv_cache *out);
/* RotatingKVCache.temporallyOrderedKV (KVCache.swift:876-887) and
 * KVCacheSimple.readKV (:516-525): K/V in temporal order, trimmed to offset,
 * without changing the cache state. */
int vkv_cache_read_kv(vkv_cache cache, void *stream, vkv_array *keys, vkv_array *values);

/* Fixed-buffer device-offset caches (VKV_CACHE_COMPILABLE*).  A decode
 * step made of vkv_cache_update, vkv_cache_make_mask and attention on these
 * caches reads no value back to the host, so it can be captured in a HIP
 * graph once and replayed (the reference's compile() path).  offset and
 * state/metaState read the device counters back (synchronizing), like the
 * reference's .item(). */

/* CompilableKVCache(from:maxLength:) (CompilableKVCache.swift:62-86): a new
 * cache holding src's state (2 float arrays) at positions [0, len) of
 * zeroed max_length buffers, offset = len. */
int vkv_cache_to_compilable(vkv_cache src, int64_t max_length, void *stream, vkv_cache *out);
/* CompilableRotatingKVCache(from:) (CompilableRotatingKVCache.swift:91-150):
 * a new cache with src's keep/maxSize/step, ring index and offset, and its
 * buffers extended with zeros to maxSize. */
int vkv_cache_to_compilable_rotating(vkv_cache rotating, void *stream, vkv_cache *out);
/* CompilableTurboQuantKVCache(from:) (CompilableTurboQuantKVCache.swift:
 * 110-160): a new cache restored from tq's encoded records and window
 * (restoreCompressed), its window write position and offset copied to
 * device counters.  tq must be in the compressed phase.  In that phase
 * update writes the new tokens (cast to the unified buffers' dtype, as the
 * reference's dynamicSliceUpdate does) at the device offset, clamped so
 * they fit, advances both counters and the host offset, and returns the
 * whole unified buffers; fill-phase updates are TurboQuantKVCache's. */
int vkv_turboquant_to_compilable(vkv_cache tq, void *stream, vkv_cache *out);
/* innerState: the arrays a captured step reads and writes in place —
 * keys and values [B,H,max,D], then the counters as int32 [1] device arrays:
 * the offset (CompilableKVCache.swift:108-113), the ring index then the
 * offset (CompilableRotatingKVCache.swift:255-264), or the window write
 * position then the offset (CompilableTurboQuantKVCache.swift:286-293, the
 * unified buffers first).  `arrays` has room for 4. */
int vkv_cache_inner_state(vkv_cache cache, vkv_array *arrays, int32_t *count);

/* dynamicSliceUpdate(src, update:, start:, axes: [axis])
 * (DynamicSlice.swift:50-71): dst[..., start + i, ...] = update[..., i, ...]
 * along `axis`, in place, where start is the int32 at device address
 * `start` read by the kernel (clamped to [0, dim - update dim]).  Up to 4-D,
 * same element size, strided. */
int vkv_dynamic_slice_update(vkv_array *dst, const vkv_array *update, const int32_t *start,
                             int32_t axis, void *stream);
/* dynamicSlice(src, start:, axes: [axis], sliceSize:) (DynamicSlice.swift:
 * 21-48): out = src[..., start : start + out dim, ...] along `axis`. */
int vkv_dynamic_slice(const vkv_array *src, const int32_t *start, int32_t axis, vkv_array *out,
                      void *stream);

/* ---------------------------------------------------- paged block pool */

typedef struct vkv_pool_params {
  int32_t num_blocks;   /* pool size in blocks (block 0 is reserved as the
                           null sentinel, PagedCacheManager.swift:86-92) */
  int32_t block_size;   /* tokens per block */
  int32_t n_layers;
  int32_t n_kv_heads;
  int32_t head_dim;
  int32_t v_head_dim;   /* 0 = head_dim; keys-only pools ignore it */
  int32_t dtype;        /* element dtype of appended K/V (and of scales) */
  int32_t bits;         /* 0 = float blocks, 4/8 = affine quantized blocks */
  int32_t group_size;   /* 64 */
  int32_t flags;        /* VKV_VIEW_KEYS_ONLY for an MLA latent pool */
} vkv_pool_params;

int vkv_pool_create(const vkv_pool_params *params, vkv_pool *out);
int vkv_pool_destroy(vkv_pool pool);
/* Bytes of device memory the pool holds. */
int vkv_pool_bytes(vkv_pool pool, int64_t *bytes);
/* Build the attention view of one layer over caller block tables. */
int vkv_pool_view(vkv_pool pool, int32_t layer, const int32_t *block_table,
                  int32_t table_stride, const int32_t *seq_lens, int32_t n_seqs,
                  int32_t max_len, vkv_paged_view *out);

/* Scatter new tokens into pool blocks (quantizing on the way for affine
 * pools).  keys [N,Hkv,D], values [N,Hkv,Dv] (strided; a [1,H,T,D] cache
 * array is passed as [T,H,D] with strides {D, T*D, 1}); slot_mapping
 * device int32 [N], slot = block_id * block_size + offset_in_block (a
 * negative slot, or one at or past num_blocks * block_size, skips its token
 * rather than writing outside the pool).  Replaces
 * the reference's per-sequence slice assignment (KVCache.swift:498-502,
 * :1105-1116) and block split (CacheCoordinator.swift:1238-1272).  Quantized
 * codes, scales and biases are bit-exact with the reference quantizer. */
int vkv_paged_append(vkv_pool pool, int32_t layer, const vkv_array *keys,
                     const vkv_array *values, const int32_t *slot_mapping, int64_t n_tokens,
                     void *stream);

/* Gather (dequant-on-read) into contiguous arrays keys [n_seqs,Hkv,T,D],
 * values [n_seqs,Hkv,T,Dv] (T = view max_len; tokens past a sequence's
 * length are left untouched), in the view's dtype.  restoreLayerData's
 * concatenation (CacheHelpers.swift:431-552) without the copies. */
int vkv_paged_gather(const vkv_paged_view *kv, vkv_array *keys, vkv_array *values,
                     void *stream);
/* Gather the raw affine codes into the reference layout: out[0..5] =
 * keys wq [n,H,T,D*bits/32] u32, keys scales, keys biases [n,H,T,D/g],
 * values wq, scales, biases (keys-only views fill out[0..2]). */
int vkv_paged_gather_quantized(const vkv_paged_view *kv, vkv_array *out, void *stream);
/* Copy whole blocks (all layers): dst[i] <- src[i] (host arrays of block
 * ids); copy-on-write of a shared partial block and the store copy of the
 * prefix cache. */
int vkv_pool_copy_blocks(vkv_pool pool, const int32_t *src, const int32_t *dst, int32_t n,
                         void *stream);

/* ------------------------------------------ prefix cache (PagedCacheManager) */

/* PagedCacheManager(blockSize:maxBlocks:modelKey:) (PagedCacheManager.swift:
 * 80-96).  model_key may be NULL.  `pool` may be NULL (bookkeeping only);
 * when given, block ids are pool block ids and stores copy KV on device. */
int vkv_prefix_create(int32_t block_size, int32_t max_blocks, const char *model_key,
                      vkv_pool pool, vkv_prefix *out);
int vkv_prefix_destroy(vkv_prefix mgr);
/* allocateBlock (:104-127): *block = -1 when the pool is exhausted. */
int vkv_prefix_allocate(vkv_prefix mgr, int32_t *block);
/* freeBlock (:135-156). */
int vkv_prefix_free(vkv_prefix mgr, int32_t block);
/* CacheCoordinator.release(blocks:) (Cache/CacheCoordinator.swift:351-358):
 * frees `blocks` leaves first (reverse order) so roots stay the newest LRU
 * entries. */
int vkv_prefix_release(vkv_prefix mgr, const int32_t *blocks, int32_t n);
/* Extra reference for a block shared by another sequence (fork). */
int vkv_prefix_incref(vkv_prefix mgr, int32_t block);
int vkv_prefix_ref_count(vkv_prefix mgr, int32_t block, int32_t *ref_count);
/* findCachedBlock(hash:) (:164-180): *block = -1 on a miss. */
int vkv_prefix_find(vkv_prefix mgr, const char *hash, int32_t *block);
/* registerBlock(_:hash:) (:187-192). */
int vkv_prefix_register(vkv_prefix mgr, int32_t block, const char *hash);
/* clear() (:195-217). */
int vkv_prefix_clear(vkv_prefix mgr);
/* storeTokenSequence(tokens:layerData:mediaSalt:) (:229-310).  Chunks
 * [0, n_data_chunks) have KV; with a pool, chunk i's KV is copied on
 * `stream` from pool block src_blocks[i] into the newly allocated block. */
int vkv_prefix_store(vkv_prefix mgr, const int64_t *tokens, int64_t n_tokens,
                     const char *media_salt, int32_t n_data_chunks,
                     const int32_t *src_blocks, void *stream);
/* fetchPrefix(tokens:mediaSalt:) (:320-376): pins and returns the matched
 * blocks (up to `capacity`), *n_blocks and *matched_tokens (0 = nil). */
int vkv_prefix_fetch(vkv_prefix mgr, const int64_t *tokens, int64_t n_tokens,
                     const char *media_salt, int32_t *blocks, int32_t capacity,
                     int32_t *n_blocks, int64_t *matched_tokens);

/* Copy-on-write before writing into `block` (the partially filled last block
 * of a fetched prefix, PagedCacheManager.swift:351-361, or a block forked to
 * several sequences with vkv_prefix_incref).  *out_block = block when the
 * caller holds the only reference and no cache entry names it; otherwise a
 * fresh block (allocated from the LRU head, evicting as allocateBlock does)
 * receives a device copy of every layer of `block` on `stream`, the
 * caller's reference moves to it (`block` keeps its cache entry and its
 * other holders), and *out_block is the fresh block (refcount 1, no cache
 * entry); -1 when no block is free.  The caller then points its block
 * table at *out_block.  Replaces the copy of every restored block the
 * reference makes (Cache/CacheHelpers.swift:431-552): only the block that
 * is written into is copied. */
int vkv_prefix_writable(vkv_prefix mgr, int32_t block, void *stream, int32_t *out_block);

/* CacheStats (PagedCacheManager.swift:10-17). */
typedef struct vkv_prefix_stats {
  int64_t total_blocks, allocated_blocks, free_blocks, cache_hits, cache_misses, evictions;
} vkv_prefix_stats;
int vkv_prefix_stats_get(vkv_prefix mgr, vkv_prefix_stats *out);
/* Block metadata: token count of a stored block (-1 if none). */
int vkv_prefix_block_tokens(vkv_prefix mgr, int32_t block, int32_t *n_tokens);

/* CacheBlock.computeBlockHash (CacheBlock.swift:110-146): SHA-256 over
 * modelKey UTF-8, "|media:" + salt, parent hash UTF-8, then the tokens as
 * raw little-endian Int64 bytes; 64 lowercase hex chars + NUL into out[65]. */
int vkv_block_hash(const char *parent_hash, const int64_t *tokens, int64_t n_tokens,
                   const char *model_key, const char *media_salt, char *out);

/* ------------------------------------------------------ on-disk formats */

/* savePromptCache(url:cache:metadata:) (MLXLMCommon/KVCache.swift:1620-1680):
 * a safetensors file with each cache's state arrays as "i.j", its metaState
 * strings as metadata "0.i.j", the user metadata as "1.<key>" and the class
 * names ("KVCache", "RotatingKVCache", "QuantizedKVCache") as "2.i", the
 * Python mlx-lm layout.  The states are copied to the host on `stream`. */
int vkv_prompt_cache_save(const char *path, const vkv_cache *caches, int32_t n_caches,
                          const char *const *meta_keys, const char *const *meta_values,
                          int32_t n_meta, void *stream);
/* loadPromptCache(url:) (:1687-1780): new cache handles into caches[0..n),
 * *n_caches = n (with caches == NULL only counts); user metadata as
 * NUL-separated key, value pairs in meta_buf (*n_meta pairs; NULL buf only
 * counts).  Errors as the reference throws them ("Unknown cache class",
 * "Mismatch in cache counts", RotatingKVCache maxSize None); the whole file
 * is validated before any cache is built.  Quantized layers keep the group
 * size and bits their metaState records (the reference rebuilds them as
 * QuantizedKVCache() and sets only the offset). */
int vkv_prompt_cache_load(const char *path, void *stream, vkv_cache *caches, int32_t capacity,
                          int32_t *n_caches, char *meta_buf, int64_t meta_buf_len,
                          int32_t *n_meta);
/* The same file written from one sequence's pool blocks (host block ids,
 * tokens 0 .. n_tokens-1 at blocks[t / block_size]): per pool layer, an
 * affine pool gives the QuantizedKVCache arrays (the stored codes, no
 * requantization), a float pool KVCacheSimple's keys and values. */
int vkv_prompt_cache_save_paged(const char *path, vkv_pool pool, const int32_t *blocks,
                                int32_t n_blocks, int64_t n_tokens,
                                const char *const *meta_keys, const char *const *meta_values,
                                int32_t n_meta, void *stream);
/* ... and read back into one sequence's pool blocks (restoreLayerData,
 * Cache/CacheHelpers.swift:431-552, without the concatenated copy): float
 * layers are appended (quantized for an affine pool), quantized layers with
 * the pool's group size and bits are written as they are, others are
 * dequantized and appended.  *n_tokens receives the token count. */
int vkv_prompt_cache_load_paged(const char *path, vkv_pool pool, const int32_t *blocks,
                                int32_t n_blocks, int64_t *n_tokens, char *meta_buf,
                                int64_t meta_buf_len, int32_t *n_meta, void *stream);

/* DiskCache.hashTokens (Cache/DiskCache.swift:659-682): the first 32 hex
 * digits of SHA-256(model key, "|media:" + salt, tokens as little-endian
 * Int64), the disk tier's file name; 32 chars + NUL into out[33]. */
int vkv_disk_hash_tokens(const int64_t *tokens, int64_t n_tokens, const char *model_key,
                         const char *media_salt, char *out);
/* TQDiskSerializer.serialize, format version 2 (Cache/TQDiskSerializer.swift:
 * 240-330): __jang_cache_format_version__ = [2], __layer_kind_i__ per layer
 * (2 kv: kv_i_keys/values; 6 rotating: rot_i_keys/values + __rot_i_meta__
 * [keep, maxSize, step, offset, idx]; 5 quantized: qkv_i_k +
 * __qkv_i_count__/_offset__/_group_size__/_bits__; 4 skip for an empty
 * cache), scalars as 1-element int32 arrays, file metadata {"format": "mlx"}
 * (DiskCache.swift:315). */
int vkv_disk_cache_save(const char *path, const vkv_cache *caches, int32_t n_caches,
                        void *stream);
/* deserializeV2 (:1023-1170) for those kinds: caches[i] = layer i's new
 * cache, NULL for a skipped layer; *n_layers = the layer count (caches ==
 * NULL only counts).  A gap in the kind tags, an incomplete payload or a
 * kind this library does not hold (TurboQuant, Mamba, composite) fails the
 * whole record, the reference's required miss. */
int vkv_disk_cache_load(const char *path, void *stream, vkv_cache *caches, int32_t capacity,
                        int32_t *n_layers);

/* Strided copy between two arrays of the same shape and element size
 * (materializes a view returned by a cache into caller memory).  Replaces
 * the reference's `x * 1` owned copy (KVCache.swift:100-102). */
int vkv_array_copy(const vkv_array *src, vkv_array *dst, void *stream);

/* Attention workspace of a stream (no reference counterpart; the reference
 * allocates per op through MLX's allocator).  The attention calls keep one
 * split-K workspace per (device, stream) that only grows; an outgrown
 * buffer is kept, not freed, because a HIP graph captured earlier on that
 * stream still points at it, and growth during capture is refused (run the
 * call once before capturing).  vkv_workspace_release frees the stream's
 * workspace on the current device and every outgrown buffer (*bytes,
 * optional, receives the total); call it only when no captured graph that
 * used the stream will be replayed again. */
int vkv_workspace_release(void *stream, int64_t *bytes);

/* ------------------------------------------------------- dispatch options */

/* Process-wide dispatch options, with no counterpart in the reference (a
 * tuning and testing aid): GENERIC_ATTENTION (0/1) sends every attention
 * call to the generic VALU kernel; DECODE_WAVES (0 = choose per launch)
 * sets the paged decode kernel's wave count; MLA_SPLITS (0 = choose) sets
 * the MLA kernel's token splits; FDECODE_WAVES (0 = choose) the float
 * decode kernel's target wave count; GATHER_TOKENS (0 = choose) the key
 * window of a multi-token chunk over a quantized or paged cache (its K/V are
 * gathered to the dtype one window at a time; by default a window's copy
 * stays within 256 MiB); REFERENCE_SOFTMAX (0/1) computes quantized
 * attention with the reference's own roundings: scores stored in the query
 * dtype, softmax(precise: false) with its AccT = T arithmetic in a pass of
 * its own (KVCache.swift:1982, mlx-generated/metal/softmax.h:10-190),
 * weights stored in the dtype, then P.V (with it off, the softmax of the
 * stored scores runs in fp32 inside one pass); SEPARATE_TOKEN_WRITE (0/1)
 * makes vkv_attention_with_cache_update's one-token step over a
 * QuantizedKVCache write the token in a launch of its own before the
 * attention (by default the matrix-core decode launch quantizes and stores
 * it as it starts; both give the same bits).  Initial values come from
 * the environment variables VKV_GENERIC_ATTENTION, VKV_DECODE_WAVES,
 * VKV_MLA_SPLITS, VKV_FDECODE_WAVES, VKV_GATHER_TOKENS,
 * VKV_REFERENCE_SOFTMAX and VKV_SEPARATE_TOKEN_WRITE, read once; calls read
 * the options, never the environment. */
enum {
  VKV_OPTION_GENERIC_ATTENTION = 0,
  VKV_OPTION_DECODE_WAVES = 1,
  VKV_OPTION_MLA_SPLITS = 2,
  VKV_OPTION_FDECODE_WAVES = 3, /* 0 = 2048: waves the float decode kernel aims for */
  VKV_OPTION_GATHER_TOKENS = 4, /* 0 = a 256 MiB copy: key window of a gathered chunk */
  VKV_OPTION_REFERENCE_SOFTMAX = 5, /* quantized attention with the reference's arithmetic */
  VKV_OPTION_SEPARATE_TOKEN_WRITE = 6, /* the router's quantized decode token in its own launch */
  VKV_OPTION_COUNT = 7
};
int vkv_set_option(int32_t which, int64_t value);
int vkv_get_option(int32_t which, int64_t *value);

/* ------------------------------------------------------- kernel timing */

/* Kernel timing, a measurement aid with no counterpart in the reference:
 * while enabled, the paged decode attention launcher (kind 0: its
 * matrix-core decode kernel, without the split-K merge), the MLA launcher
 * (kind 1: its attention kernel) and the dense float decode launcher (kind
 * 2: its decode kernel, without the merge) and the TurboQuant launchers
 * (kind 3: the key encode kernel, kind 4: the key decode kernel) and the
 * affine pool append (kind 5: its quantize-and-store kernel) launch
 * that kernel with a start/stop HIP event pair (hipExtLaunchKernel),
 * recorded at the kernel's own start and end.  vkv_kernel_timing_read waits
 * for the launches of a kind recorded so far and returns their total
 * milliseconds and count, then forgets them. */
enum { VKV_TIME_DECODE = 0, VKV_TIME_MLA = 1, VKV_TIME_FDECODE = 2, VKV_TIME_TQ_ENCODE = 3,
       VKV_TIME_TQ_DECODE = 4, VKV_TIME_APPEND = 5 };
int vkv_kernel_timing(int32_t enable);
int vkv_kernel_timing_read(int32_t kind, double *total_ms, int32_t *count);

/* ------------------------------------------------------------ synthetic */

/* Fill a contiguous f16/bf16/f32 device buffer with counter-based normal
 * samples (SplitMix64 -> Box-Muller in fp32 -> round to dtype), value i
 * depends only on (seed, i).  `std` scales the samples.  Benchmark input
 * generator; no reference counterpart. */
int vkv_fill_normal(void *data, int32_t dtype, int64_t n, uint64_t seed, float std,
                    void *stream);

#ifdef __cplusplus
}
#endif
#endif /* VKV_H */
