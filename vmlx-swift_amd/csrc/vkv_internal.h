// vkv_internal.h -- kernel argument blocks and launchers shared by the host
// code (vkv_capi.cpp) and the HIP kernels (vkv_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <stdexcept>
#include <string>

namespace vkv {

struct Error : std::runtime_error {
  explicit Error(const std::string& m) : std::runtime_error(m) {}
};

#define VKV_CHECK(cond, msg)                                      \
  do {                                                            \
    if (!(cond)) throw ::vkv::Error(std::string(msg));            \
  } while (0)

#define VKV_HIP(call)                                                              \
  do {                                                                             \
    hipError_t e_ = (call);                                                        \
    if (e_ != hipSuccess)                                                          \
      throw ::vkv::Error(std::string(#call) + ": " + hipGetErrorString(e_));       \
  } while (0)

inline int elem_bytes(int dtype) { return dtype == 0 ? 4 : 2; }

// Rows of a strided tensor whose last dim (D) is contiguous.  Row r is
// (i0, i1, i2) with r = (i0 * e1 + i1) * e2 + i2; strides in elements.
struct RowSrc {
  const void* ptr;
  int64_t e0, e1, e2;
  int64_t s0, s1, s2;
};

// Where quantized / float rows land.
struct RowDst {
  // reference layout (mode 0): contiguous wq [rows][D*bits/32], scales and
  // biases [rows][D/group]; float copy (mode 0, bits 0): out [rows][D].
  void* wq;
  void* scales;
  void* biases;
  // paged (mode 1): chunk = base + block * block_bytes + head * head_bytes.
  uint8_t* base;
  int64_t block_bytes, head_bytes;
  int32_t block_size;
  int32_t is_v;              // V rows (affine: dim-major codes)
  int32_t c_off;             // codes (or float values) of this matrix in a chunk
  int32_t s_off;             // affine: scale/bias area of the chunk
  int32_t G;                 // affine: groups per row
  int32_t keys_only;         // affine: chunk holds keys only (MLA latent)
  // slot of token n (n = row / e2 for paged rows ordered (token, head)):
  const int32_t* slots;      // explicit [N] (slot = block*bs + offset; slots at
                             //   or past slot_limit, when set, are skipped), or
  const int32_t* table;      // block table [e0][table_stride] with
  int32_t table_stride;      //   token n -> (b = n / seq_S, pos = start + n % seq_S)
  int32_t seq_S, start;
  int64_t slot_limit;        // explicit slots: the pool's slot count (0 = unchecked)
};

// One component (codes, scales, biases, or float values) of K or V.
// Dense: byte address of (seq s, head h, token t) = ptr + s*sb + h*sh + t*st.
// Paged: ptr + block*sb + h*sh + t_in_block*st, block from the table.
struct Comp {
  const uint8_t* ptr;
  int64_t sb, sh, st;
};

struct KVSrc {
  Comp kc, ks, kb, vc, vs, vb;  // dense layouts and float blocks
  const int32_t* table;   // nullptr = dense
  int32_t table_stride;
  int32_t block_size;
  const int32_t* seq_lens;  // nullptr = every row has T tokens
  int32_t T;
  // Affine paged chunks (qfmt != 0): chunk = base + block*block_bytes +
  // head*head_bytes, codes/scale-bias addressed by the chunk format.
  int32_t qfmt;
  const uint8_t* base;
  int64_t block_bytes, head_bytes;
  int32_t kc_off, vc_off, sb_off;
  int32_t G, keys_only, D;
};

struct AttnArgs {
  const void* q;
  int64_t q_sb, q_sh, q_sl;  // element strides of q (batch row, head, l)
  int32_t L, Hq, Hkv, D, Dv;
  float scale;
  KVSrc kv;
  int32_t mask_mode;       // 0 none, 1 causal, 2 bool array, 3 additive array
  int32_t mask_dtype;      // additive mask element type (0 f32, 1 f16, 2 bf16)
  const void* sinks;       // per query head attention sink logits [Hq], or null
  int32_t sinks_dtype;     // (0 f32, 1 f16, 2 bf16)
  const void* mask;
  int64_t m_sb, m_sh, m_sl, m_st;
  void* out;
  int64_t o_sb, o_sh, o_sl;
  int32_t part_tokens, n_parts;
  // prefill over a window of the keys (0, 0 = all parts): this launch runs
  // parts part0 .. part0 + parts_run - 1 of n_parts, over K/V whose first row
  // is token t_base
  int32_t part0, parts_run, t_base;
  float* ws_o;             // [rows][Hq][n_parts][Dv]
  float* ws_ml;            // [rows][Hq][n_parts][2] (max, sum)
  int32_t group;           // affine quantization group (0 = 64)
  // float decode only: key/value row new_t of every (batch row, kv head)
  // comes from these source rows (byte strides) instead of the cache, and
  // the kernel writes it into the cache (a cache update's deferred token)
  int32_t has_new;
  int64_t new_t;
  const uint8_t* nk_ptr;
  const uint8_t* nv_ptr;
  int64_t nk_sb, nk_sh, nv_sb, nv_sh;
  // float decode only: one zeroed counter per (batch row, kv head, head
  // group); non-null merges the split partials inside the decode launch
  // (the last part of a row merges, then zeroes its counter again)
  uint32_t* counters;
  // float decode only: > 0 = the launch is one workgroup of wg_parts waves
  // per (row, kv head, head group) (n_parts == wg_parts), merged in LDS
  int32_t wg_parts;
};

// Quantized attention with the reference's arithmetic (vkv_refattn.hip):
// scores stored in the query dtype, the reference softmax (AccT = T) in its
// own pass, then P.V.  One launch covers the query positions
// [l0, l0 + nl) of every batch row.
constexpr int kMaxRefD = 256;
struct RefArgs {
  AttnArgs a;
  int32_t group, bits;
  int32_t deq_round;       // K/V dequantized to the dtype first (the tiled matmul path)
  int32_t score_f32;       // an f32 additive mask: f32 scores, fp32 softmax, f32 weights
  int32_t l0, nl;
  float* sc;               // scores, then weights: [B][Hq][nl][tpad]
  int64_t tpad;
  int32_t n_parts, part_tokens;
  float* ws;               // P.V partials [n_parts][n_rows][Dv] (n_parts > 1)
  int64_t n_rows;          // B * Hq * nl
};
size_t ref_scores_lds(int D);
size_t ref_pv_lds(int Dv);
// P.V token split for a launch; returns the part length (a multiple of 64)
int ref_part_tokens(int64_t B, int Hkv, int nrows, int64_t T, int* n_parts);
void launch_ref_attention(int dtype, const RefArgs& r, int64_t B, hipStream_t st);
// The reference softmax in place over bf16 score rows (row r holds
// seq_lens[r / per_b] scores, or T when seq_lens is null).
void launch_ref_softmax_bf16(uint16_t* sc, int64_t rows, int64_t tpad, const int32_t* seq_lens,
                             int32_t T, int64_t per_b, hipStream_t st);

// ---- launchers (vkv_kernels.hip) ----
void launch_quantize_rows(int dtype, int bits, int group, int mode, const RowSrc& src,
                          const RowDst& dst, int64_t rows, int D, hipStream_t st);
void launch_copy_rows(int dtype, int mode, const RowSrc& src, const RowDst& dst, int64_t rows,
                      int D, hipStream_t st);
// Paged append of ntok tokens x H heads of K (and V when with_v) in one
// launch; rows of the sources are (token, head), D = head dim of both.
bool append_affine_supported(int bits, int group, int D);
void launch_append_affine(int dtype, int bits, int group, const RowSrc& sk, const RowSrc& sv,
                          const RowDst& dk, const RowDst& dv, int64_t ntok, int H, int D, bool with_v,
                          hipStream_t st);
void launch_dequantize(int dtype, int bits, int group, const uint32_t* wq, const void* scales,
                       const void* biases, void* out, int64_t rows, int D, hipStream_t st);
// Gather rows of paged/dense KV into dense arrays.  which: 0 = keys, 1 = values.
// out_kind: 0 = values in dtype (dequantized when bits > 0), 1 = reference
// layout codes (+ scales, biases).
struct GatherArgs {
  KVSrc kv;
  int32_t n_seqs, H, T, D, which, bits, group, dtype;
  int32_t t_begin;  // first token gathered: output token t is token t_begin + t
  void* out;        // [n,H,T,D] values, or [n,H,T,D*bits/32] u32 codes
  void* out_s;      // [n,H,T,D/group]
  void* out_b;
  void* out_v;      // values (out_kind 0): non-null gathers K into out and V
                    //   into out_v in one call (which is then ignored)
  int32_t out_cap;  // codes (out_kind 1): tokens per (seq, head) row of the
  int32_t out_t0;   //   outputs (0 = T) and the output token of gathered token 0
};
void launch_gather(const GatherArgs& g, int out_kind, hipStream_t st);
// Strided 4-D copy (element size 2 or 4): dst[i] = src[i].
void launch_copy4d(int esize, const void* src, const int64_t* shape, const int64_t* sstr,
                   void* dst, const int64_t* dstr, hipStream_t st);
// One strided 4-D copy (element strides) for launch_copy4d_pair.
struct Copy4D {
  const void* src;
  void* dst;
  int64_t n[4], s[4], d[4];
};
// Two copies of one element size in one launch.
void launch_copy4d_pair(int esize, const Copy4D& c0, const Copy4D& c1, hipStream_t st);
void launch_fill_normal(int dtype, void* data, int64_t n, uint64_t seed, float std,
                        hipStream_t st);
void launch_attention(int dtype, int bits, int group, bool quant_semantics,
                      const AttnArgs& a, int64_t rows, hipStream_t st);
// The split-K merge of launch_attention's partials (a.n_parts > 1).
void launch_attn_combine(int dtype, const AttnArgs& a, int64_t rows, hipStream_t st);
// One-token decode over dense float K/V (vkv_fdecode.hip): whether a call
// qualifies (float, L = 1, dense, D = Dv in {64, 128, 256}, 16-byte aligned
// rows), its token split (about 2048 waves, 64-token steps), and the launch
// (with the merge when a.n_parts > 1).
// Multi-query attention (L >= 2) over dense bf16 / f16 K/V, D = 128, no or
// causal mask, on matrix cores (vkv_prefill.hip).
bool prefill_supported(int dtype, int bits, const AttnArgs& a);
int prefill_parts(int64_t batch, int Hkv, int64_t L, int rep, int64_t T, int D, int32_t* part_tokens);
// combine = false leaves the split merge to the caller (a window of parts)
void launch_prefill(int dtype, bool qsem, const AttnArgs& a, int64_t batch, hipStream_t st,
                    bool combine = true);
bool fdecode_supported(int dtype, int bits, bool qsem, const AttnArgs& a);
int fdecode_parts(int64_t rows_x_heads, int64_t T, int32_t* part_tokens, int waves);
void launch_fdecode(int dtype, const AttnArgs& a, int64_t rows, hipStream_t st);
// counters per batch row the float decode's in-launch merge uses, and
// whether a launch merges inside (a small merge) or in attn_combine_kernel
int fdecode_counter_count(int Hq, int Hkv);
bool fdecode_merge_here(int n_parts, int Dv, int Hq, int Hkv);
// parts of a workgroup-per-row launch (0: not a small launch), and their tokens
int fdecode_wg_parts(int64_t rows, int Hq, int Hkv, int64_t T, int D, int dtype,
                     int32_t* part_tokens);
// MFMA decode attention over paged affine bf16 KV (vkv_decode.hip).
struct DecodeArgs {
  const uint16_t* q;         // [n_seqs][Hq][D] bf16 / f16
  int64_t q_ss, q_sh;        // element strides
  uint16_t* out;             // [n_seqs][Hq][D] bf16 / f16
  int64_t o_ss, o_sh;
  float scale;
  const uint8_t* base;       // layer base of the chunk pool
  int64_t block_bytes, head_bytes;
  int32_t kc_off, vc_off, sb_off;
  const int32_t* table;
  int32_t table_stride;
  int32_t block_size;        // tokens per pool block (a multiple of 32)
  const int32_t* seq_lens;   // nullptr = every sequence holds max_len tokens
  int32_t max_len;
  int32_t Hq, Hkv, rep;
  int32_t n_seqs;
  int32_t n_waves;           // decode waves per launch (0 = choose)
  float* ws;                 // split-K workspace, qdecode_workspace_floats floats
  float* ws_o;               // set per launch: partial outputs [slot][head][D]
  float* ws_ml;              //                 partial (max, sum) [slot][head][2]
  int32_t ws_hdr;            //   then (as int32 at ws_ml + ws_hdr) the number
                             //   of partials of each (sequence, head pair)
  int32_t max_parts;         // set per launch: partials per (sequence, head pair), at most
  int32_t dtype;             // kBF16 or kF16: queries, scales / biases and output
  int32_t group;             // quantization group: 64, or 128 (fused mode, D >= 128)
  uint16_t* sc;              // reference path: bf16 score / weight rows
  int64_t sc_stride;         //   [n_seqs][Hq][sc_stride], sc_stride >= max_len, % 64 == 0
  uint32_t* counters;        // zeroed per-pair counters: the partials merge inside the
                             //   decode launch (nullptr: in qdecode_combine_kernel)
  // the router's decode token (nullptr: none): the key / value rows
  // [seq][kv head][D] of each sequence's last token, quantized and stored
  // into its block by the launch itself (fused mode); element strides
  const uint16_t* new_k;
  const uint16_t* new_v;
  int64_t nk_ss, nk_sh, nv_ss, nv_sh;
};
bool qdecode_supported(int dtype, int bits, int D, int block_size, int rep, int group);
// (sequence, kv head) pairs are split into head groups of 4 or 8 query heads
int qdecode_head_groups(int rep);
// sequences per launch, at most (larger batches are launched in slices)
int qdecode_max_seqs();
// longest sequence (tokens) the matrix-core decode takes
int qdecode_max_len();
// decode waves for a launch of n_seqs sequences (want > 0 overrides)
int qdecode_waves(int n_seqs, int Hkv, int rep, int max_len, int want);
size_t qdecode_workspace_floats(int n_seqs, int Hkv, int rep, int D, int max_len);
// ref: the reference-arithmetic path (score rows, the reference softmax,
// P.V from the stored weights) in place of the fused single pass
void launch_qdecode(const DecodeArgs& a, int bits, int D, hipStream_t st, bool ref = false);
// Scratch of the no-allocation decode entry point: a fixed device array in
// vkv_decode.hip, of decode_scratch_bytes() bytes per device.  Returns its
// device address on the current device (resolved once per device), or
// throws when `floats` does not fit.
float* decode_scratch(size_t floats);
size_t decode_scratch_bytes();

// Absorbed-latent MLA decode over a keys-only 8-bit paged view (vkv_mla.hip):
// 576-dim entries (512 latent + 64 rope), values = the first 512 dims, one
// kv head, queries and output bf16.
struct MlaArgs {
  const uint16_t* q;         // [n_seqs, H, 576] bf16
  int64_t q_ss, q_sh;        // element strides (sequence, head)
  uint16_t* out;             // [n_seqs, H, 512] bf16
  int64_t o_ss, o_sh;
  float scale;
  const uint8_t* base;       // block 0 of the layer
  int64_t block_bytes;
  int32_t sb_off;            // scale/bias area offset within a chunk
  const int32_t* table;
  int32_t table_stride, block_size;
  const int32_t* seq_lens;   // nullptr = every sequence holds max_len
  int32_t max_len, H, n_seqs;
  int32_t n_splits, split_len;  // token splits per sequence and their length
  uint16_t* ws_o;            // split partials o/l (bf16) [seq][split][head][512]
  float* ws_ml;              //                (max, sum) [seq][split][head][2]
};
bool mla_supported(int dtype, int bits, int group, int head_dim, int v_head_dim, int n_kv_heads,
                   int block_size);
// Token splits for a launch (want > 0 overrides); sets a.n_splits and
// a.split_len and returns the workspace floats the launch needs.
// The chunk geometry the kernel's 16-byte raw-tile loads need.
bool mla_layout_supported(const uint8_t* base, int64_t block_bytes, int64_t sb_off);
size_t mla_plan(MlaArgs& a, int want);
void launch_mla(const MlaArgs& a, hipStream_t st);

// ---- device-offset operations (vkv_compile.hip)
// A copy of a block of up to 4 dims whose start along `axis` is the int32
// at `start` (device memory), clamped to [0, limit - shape[axis]]: on the
// destination side for a slice update, on the source side for a slice.
struct DynCopy {
  const uint8_t* src;
  int64_t sstr[4];     // element strides
  uint8_t* dst;
  int64_t dstr[4];
  int64_t shape[4];    // the copied block
  int32_t axis;
  int32_t on_dst;      // 1: dst index += start (update); 0: src index += start (slice)
  int64_t limit;       // extent of the offset side along axis
  const int32_t* start;
};
void launch_dyn_copy(int esize, const DynCopy& c, hipStream_t st);
// Write counters of the fixed-buffer caches: ctr[0] = offset, ctr[1] = ring
// write index.  Advance by n (with the ring wrap when ring != 0), or set.
void launch_counter_advance(int32_t* ctr, int n, int ring, int max_size, int keep, hipStream_t st);
void launch_counter_set(int32_t* ctr, int32_t offset, int32_t idx, hipStream_t st);
// ctr[0] += n and ctr[1] += n (offset and window write position).
void launch_counter_advance_both(int32_t* ctr, int n, hipStream_t st);
// [n, cols] bool mask from the device offset (see vkv_compile.hip).
void launch_offset_mask(const int32_t* ctr, int n, int cols, int window, int ring, uint8_t* mask,
                        hipStream_t st);
// [n, off + n] causal bool mask with a host offset (and window when > 0).
void launch_causal_mask(int n, int64_t off, int window, uint8_t* mask, hipStream_t st);
// [size] bool: roll(arange(size) >= size - window, shift).
void launch_roll_mask(int64_t size, int64_t window, int64_t shift, uint8_t* mask, hipStream_t st);
// ---- TurboQuant codec (vkv_tq.hip) ----
constexpr int kTqTileRows = 32;  // vectors per workgroup tile
// The power-of-two blocks of TQHadamard.decomposePow2Blocks and their f32
// 1 / sqrt(n) scales.
struct TqBlocks {
  int32_t n;
  int32_t size[16], off[16];
  float scale[16];
};
struct TqEncodeArgs {
  const void* x;             // [B, H, T, D] strided source, element strides
  int32_t dtype;
  int64_t sb, sh, st;
  int32_t B, H, Tc, t0, D;   // encodes tokens [t0, t0 + Tc)
  const float* signs;        // [D] rotation signs
  const float* codebook;     // [nc] levels
  const float* bounds;       // [nc - 1] midpoints
  int32_t nc, bits;          // levels, index bits
  const float* St;           // keys: S transposed [D][D]; null for values
  TqBlocks blocks;
  uint32_t* indices;         // packed codes (zeroed first)
  uint32_t* qjl;             // packed signs (keys, zeroed first)
  uint16_t* vec_norms;       // f16 [rows]
  uint16_t* res_norms;       // f16 [rows] (keys)
};
struct TqDecodeArgs {
  const uint32_t* indices;
  const uint32_t* qjl;       // keys; null for values
  const uint16_t* vec_norms;
  const uint16_t* res_norms;
  int32_t B, H, Tc, D, bits;
  const float* codebook;
  const float* signs;
  const float* S;            // keys: [D][D]; null for values
  float qs;                  // f32(sqrt(pi / 2)) / f32(D)
  TqBlocks blocks;
  void* out;                 // f16 or f32, element strides, tokens from t0
  int32_t out_dtype, t0;
  int64_t osb, osh, ost;
};
void launch_tq_encode(const TqEncodeArgs& a, hipStream_t st);
void launch_tq_decode(const TqDecodeArgs& a, hipStream_t st);
// Zeros in `rows` runs of run_bytes, pitch_bytes apart (2-byte units).
void launch_zero_runs(void* base, int64_t pitch_bytes, int64_t run_bytes, int64_t rows,
                      hipStream_t st);
// dst = src with a dtype conversion (4-D, element strides).
void launch_cast4d(const void* src, int sdt, const int64_t* shape, const int64_t* sstr, void* dst,
                   int ddt, const int64_t* dstr, hipStream_t st);

// createBatchCausalMask: [batch, 1, n, cols] bytes from host per-slot
// offsets and key lengths; window < 0 means none.
constexpr int kBatchMaskSlots = 240;
void launch_batch_mask(int n, int cols, int window, const int32_t* offsets, const int32_t* key_lens,
                       int batch, uint8_t* mask, hipStream_t st);

// Kernel timing (a measurement aid): while enabled, launchers start their
// main kernel with hipExtLaunchKernelGGL and a start/stop event pair, which
// the runtime records at the kernel's own start and end.
enum { kTimeDecode = 0, kTimeMla = 1, kTimeFDecode = 2, kTimeTqEncode = 3, kTimeTqDecode = 4,
       kTimeAppend = 5, kTimeKinds = 6 };
struct TimedLaunch {
  int kind = 0;
  hipEvent_t start = nullptr, stop = nullptr;  // null when timing is off
};
TimedLaunch timing_prepare(int kind);
void timing_commit(const TimedLaunch& t);  // after the launch
void timing_enable(bool on);
// Waits for the recorded launches of a kind; total milliseconds and count,
// then forgets them.
void timing_read(int kind, double* total_ms, int* count);

// Block pairs passed by value to the block-copy kernel.
struct BlockPairs {
  static constexpr int kMax = 256;
  int32_t src[kMax];
  int32_t dst[kMax];
};
// src/dst are host arrays of block ids.
void launch_copy_blocks(const uint8_t* base, int64_t layer_bytes, int n_layers,
                        int64_t block_bytes, const int32_t* src, const int32_t* dst, int n,
                        hipStream_t st);
void launch_fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t st);
// Scatter reference-layout affine rows (codes + scales + biases) into paged
// chunks: the inverse of the code gather (used by QuantizedKVCache.state=).
struct ScatterCodesArgs {
  const uint32_t* wq;       // [n,H,T,D*bits/32] contiguous
  const void* scales;       // [n,H,T,D/group]
  const void* biases;
  int32_t n_seqs, H, T, D, bits, group, dtype, is_v;
  RowDst dst;               // paged destination, slots from table (seq_S = T)
};
void launch_scatter_codes(const ScatterCodesArgs& a, hipStream_t st);

}  // namespace vkv
