// vkv_host.h -- host-side objects behind the C ABI: device buffers, the
// per-layer caches (KVCacheSimple / RotatingKVCache / QuantizedKVCache
// state machines), the paged block pool and the prefix-cache manager.
#pragma once

#include <hip/hip_runtime.h>

#include <functional>
#include <list>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/vkv.h"
#include "vkv_internal.h"

namespace vkv {

// Owned device allocation.  hipFree synchronizes the device, so a buffer can
// be dropped while work that reads it is still queued.
class DevBuf {
 public:
  DevBuf() = default;
  explicit DevBuf(size_t bytes) { alloc(bytes); }
  ~DevBuf() { release(); }
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  DevBuf(DevBuf&& o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr; o.n_ = 0; }
  DevBuf& operator=(DevBuf&& o) noexcept {
    if (this != &o) {
      release();
      p_ = o.p_;
      n_ = o.n_;
      o.p_ = nullptr;
      o.n_ = 0;
    }
    return *this;
  }
  void alloc(size_t bytes) {
    release();
    if (bytes) VKV_HIP(hipMalloc(&p_, bytes));
    n_ = bytes;
  }
  // Grow to at least `bytes` (contents are not kept); a buffer that is
  // large enough stays where it is, so views into it and work already
  // queued on it keep their address, and no hipFree stalls the device.
  void ensure(size_t bytes) {
    if (bytes > n_) alloc(bytes);
  }
  void release() {
    if (p_) (void)hipFree(p_);
    p_ = nullptr;
    n_ = 0;
  }
  void* get() const { return p_; }
  uint8_t* bytes() const { return static_cast<uint8_t*>(p_); }
  size_t size() const { return n_; }

 private:
  void* p_ = nullptr;
  size_t n_ = 0;
};

inline hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

// A dense [B,H,cap,D] float buffer with the reference's 4-D array semantics.
struct Dense4 {
  std::shared_ptr<DevBuf> buf;
  int dtype = 2;
  int64_t B = 0, H = 0, cap = 0, D = 0;
  bool empty() const { return !buf; }
  int64_t bytes_per_el() const { return elem_bytes(dtype); }
  vkv_array view(int64_t len) const;  // [B,H,len,D] over [.., cap, ..]
};

// Dense helpers shared by the caches (vkv_host.cpp).
void check4(const vkv_array& a, const char* name);
Dense4 alloc_dense(int64_t B, int64_t H, int64_t cap, int64_t D, int dtype, bool zero,
                   hipStream_t st);
// dst[:, :, dt0:dt0+len, :] = src[:, :, st0:st0+len, :] (same dtype)
void copy_tokens(const Dense4& dst, int64_t dt0, const vkv_array& src, int64_t st0, int64_t len,
                 hipStream_t st);
void copy_tokens_kv(const Dense4& dk, const Dense4& dv, int64_t dt0, const vkv_array& k,
                    const vkv_array& v, int64_t st0, int64_t len, hipStream_t st);
void copy_dense(const Dense4& dst, int64_t dt0, const Dense4& src, int64_t st0, int64_t len,
                hipStream_t st);
Dense4 dense_from_array(const vkv_array& a, hipStream_t st);

// Chunk layout shared by the pool and the quantized cache: byte sizes of one
// matrix's codes (or float values) and of the scale/bias area, the chunk
// size, and the offsets of K, V and the scale/bias area.
struct ChunkLayout {
  int64_t codes, sb, head;
  int32_t kc, vc, sbo;
};
// A paged affine destination for K (which 0) or V (which 1) rows.
RowDst affine_dst(uint8_t* base, int64_t block_bytes, int64_t head_bytes, int block_size,
                  const ChunkLayout& L, int which, int G, bool keys_only);

// Base of the per-layer caches (protocol KVCache, KVCache.swift:38-77).
class Cache {
 public:
  virtual ~Cache() = default;
  int64_t offset = 0;
  // offset as the protocol reports it (the fixed-buffer caches keep theirs
  // in device memory and read it back here)
  virtual int64_t current_offset() { return offset; }
  // BaseKVCache.offset setter (KVCache.swift:256-262)
  virtual void set_offset(int64_t v) { offset = v; }
  virtual int kind() const = 0;
  virtual int64_t max_size() const { return -1; }
  virtual bool trimmable() const { return false; }
  virtual int64_t trim(int64_t) { return 0; }
  virtual int64_t capacity() const = 0;
  virtual void update(const vkv_array&, const vkv_array&, hipStream_t, vkv_array*, vkv_array*) {
    throw Error("update(keys:values:) is not available on this cache");
  }
  virtual void update_quantized(const vkv_array&, const vkv_array&, hipStream_t, vkv_paged_view*) {
    throw Error("updateQuantized is only available on QuantizedKVCache");
  }
  virtual int state(hipStream_t, vkv_array* out) = 0;
  virtual void set_state(const vkv_array* arrays, int count, hipStream_t) = 0;
  virtual std::vector<std::string> meta_state() const { return {""}; }
  virtual void set_meta_state(const std::vector<std::string>& v);
  virtual std::unique_ptr<Cache> copy(hipStream_t) = 0;
  virtual void read_kv(hipStream_t, vkv_array* k, vkv_array* v) = 0;
  // BaseKVCache.makeMask (KVCache.swift:287-311)
  virtual int make_mask(int n, int window, bool return_array, hipStream_t st, vkv_array* mask);

  // A one-token write an update may leave to the attention that follows
  // it (the router's decode step): while armed, KVCacheSimple and
  // RotatingKVCache record the new token's copy here instead of launching
  // it, and the float decode kernel writes the token into the cache as it
  // reads it.  Whoever arms it either hands the record to that kernel or
  // calls flush_pending() before anything else reads the cache.
  struct PendingToken {
    bool set = false;
    const Dense4* dk = nullptr;
    const Dense4* dv = nullptr;
    int64_t pos = 0;           // token position in the cache buffers
    vkv_array k{}, v{};        // the new token's [B, H, 1, D] source rows
  };
  bool defer_token = false;
  PendingToken pending;
  void flush_pending(hipStream_t st);

 protected:
  // the copy of an update's new tokens into the buffers (recorded instead
  // when armed and the update is one token)
  void write_tokens(const Dense4& dk, const Dense4& dv, int64_t dt0, const vkv_array& k,
                    const vkv_array& v, int64_t len, hipStream_t st);
  DevBuf mask_buf_;
  int causal_array_mask(int n, int64_t off, int window, hipStream_t st, vkv_array* mask);
};

std::unique_ptr<Cache> make_cache(const vkv_cache_params& p);

class SimpleCache : public Cache {
 public:
  explicit SimpleCache(int step) : step_(step) {}
  int kind() const override { return VKV_CACHE_SIMPLE; }
  bool trimmable() const override { return true; }
  int64_t trim(int64_t n) override;
  int64_t capacity() const override { return k_.cap; }
  void update(const vkv_array& k, const vkv_array& v, hipStream_t st, vkv_array* ok,
              vkv_array* ov) override;
  int state(hipStream_t, vkv_array* out) override;
  void set_state(const vkv_array* a, int count, hipStream_t st) override;
  std::unique_ptr<Cache> copy(hipStream_t st) override;
  void read_kv(hipStream_t, vkv_array* k, vkv_array* v) override;
  std::unique_ptr<Cache> to_quantized(int group, int bits, hipStream_t st);
  int step_;
  Dense4 k_, v_;
};

class RotatingCache : public Cache {
 public:
  RotatingCache(int max_size, int keep, int step) : keep_(keep), max_(max_size), step_(step) {}
  int kind() const override { return VKV_CACHE_ROTATING; }
  int64_t max_size() const override { return max_; }
  bool trimmable() const override { return offset < max_; }
  int64_t trim(int64_t n) override;
  int64_t capacity() const override { return k_.cap; }
  void update(const vkv_array& k, const vkv_array& v, hipStream_t st, vkv_array* ok,
              vkv_array* ov) override;
  int state(hipStream_t, vkv_array* out) override;
  void set_state(const vkv_array* a, int count, hipStream_t st) override;
  std::vector<std::string> meta_state() const override;
  void set_meta_state(const std::vector<std::string>& v) override;
  std::unique_ptr<Cache> copy(hipStream_t st) override;
  void read_kv(hipStream_t st, vkv_array* k, vkv_array* v) override;
  int make_mask(int n, int window, bool return_array, hipStream_t st, vkv_array* mask) override;
  int64_t keep_, max_, step_;
  int64_t idx_ = 0;
  Dense4 k_, v_;
  Dense4 ordered_k_, ordered_v_;  // temporallyOrderedKV result

 private:
  void update_concat(const vkv_array& k, const vkv_array& v, hipStream_t st);
  bool update_in_place(const vkv_array& k, const vkv_array& v, hipStream_t st);
  bool can_update_in_place(int64_t S) const;
  Dense4 temporal_order(const Dense4& a, hipStream_t st) const;
  Dense4 trim_cat(int64_t trim_size, const Dense4& a, const vkv_array* append, hipStream_t st) const;
  void outputs(vkv_array* ok, vkv_array* ov) const;
};

// Fixed-buffer caches with the write position in device memory
// (CompilableKVCache.swift:40-262, BatchEngine/CompilableRotatingKVCache.
// swift:1-265): [B, H, max, D] buffers allocated once, updates written at
// the device counter by a kernel that reads it, the counters advanced on
// the device, the full buffers returned, and the mask built on the device,
// so a decode step issues no host read and can be captured in a HIP graph.
// Counters: int32 [2] = (offset, ring write index).
class CompilableCache : public Cache {
 public:
  CompilableCache(int64_t max_length, int step);
  int kind() const override { return VKV_CACHE_COMPILABLE; }
  int64_t current_offset() override { return counters().first; }
  // CompilableKVCache.offset setter (CompilableKVCache.swift:96-104)
  void set_offset(int64_t v) override;
  bool trimmable() const override { return true; }
  int64_t trim(int64_t n) override;
  int64_t capacity() const override { return k_.cap; }
  void update(const vkv_array& k, const vkv_array& v, hipStream_t st, vkv_array* ok,
              vkv_array* ov) override;
  int state(hipStream_t, vkv_array* out) override;
  void set_state(const vkv_array* a, int count, hipStream_t st) override;
  std::unique_ptr<Cache> copy(hipStream_t st) override;
  void read_kv(hipStream_t, vkv_array* k, vkv_array* v) override;
  int make_mask(int n, int window, bool return_array, hipStream_t st, vkv_array* mask) override;
  // innerState (CompilableKVCache.swift:108-113): keys, values, offset
  int inner_state(vkv_array* out);
  // CompilableKVCache(from:maxLength:) (CompilableKVCache.swift:62-86)
  void init_from(const vkv_array* state, int count, hipStream_t st);
  std::pair<int64_t, int64_t> counters() const;  // host read of (offset, idx)
  int64_t max_, step_;
  Dense4 k_, v_;
  DevBuf ctr_;
  hipStream_t last_ = nullptr;  // stream of the last device write

 protected:
  void alloc_buffers(const vkv_array& k, const vkv_array& v, int64_t len, hipStream_t st);
  std::map<int, DevBuf> masks_;  // one mask buffer per row count, never moved
};

class CompilableRotatingCache : public RotatingCache {
 public:
  CompilableRotatingCache(int max_size, int keep, int step);
  int kind() const override { return VKV_CACHE_COMPILABLE_ROTATING; }
  int64_t current_offset() override;
  void set_offset(int64_t v) override;
  int64_t trim(int64_t n) override;
  bool trimmable() const override;
  int64_t capacity() const override { return k_.cap; }
  void update(const vkv_array& k, const vkv_array& v, hipStream_t st, vkv_array* ok,
              vkv_array* ov) override;
  int state(hipStream_t, vkv_array* out) override;
  void set_state(const vkv_array* a, int count, hipStream_t st) override;
  std::vector<std::string> meta_state() const override;
  void set_meta_state(const std::vector<std::string>& v) override;
  std::unique_ptr<Cache> copy(hipStream_t st) override;
  void read_kv(hipStream_t st, vkv_array* k, vkv_array* v) override;
  int make_mask(int n, int window, bool return_array, hipStream_t st, vkv_array* mask) override;
  // innerState (CompilableRotatingKVCache.swift:255-264): keys, values,
  // ring index, offset
  int inner_state(vkv_array* out);
  // CompilableRotatingKVCache(from:) (CompilableRotatingKVCache.swift:91-150)
  void init_from(const RotatingCache& src, hipStream_t st);
  DevBuf ctr_;
  mutable hipStream_t last_ = nullptr;

 private:
  void pull() const;  // counters -> offset, idx_ (host mirrors)
  void push(hipStream_t st);
  std::map<int, DevBuf> masks_;
};

// QuantizedKVCache on paged storage: 32-token blocks, block id j*B + b for
// batch row b's j-th block, so growth never moves a block.
class QuantizedCache : public Cache {
 public:
  static constexpr int kBlock = 32;
  QuantizedCache(int group, int bits, int step) : group_(group), bits_(bits), step_(step) {}
  int kind() const override { return VKV_CACHE_QUANTIZED; }
  bool trimmable() const override { return true; }
  int64_t trim(int64_t n) override;
  int64_t capacity() const override { return cap_; }
  void update_quantized(const vkv_array& k, const vkv_array& v, hipStream_t st,
                        vkv_paged_view* out) override;
  // updateQuantized in two halves: the bookkeeping (growth, offset; returns
  // the first new token's position), then the quantized write of the new
  // tokens -- which a decode launch may do instead (vkv_decode.hip)
  int64_t advance(const vkv_array& k, const vkv_array& v, hipStream_t st);
  void write_tokens(const vkv_array& k, const vkv_array& v, int64_t prev, hipStream_t st);
  int state(hipStream_t st, vkv_array* out) override;
  void set_state(const vkv_array* a, int count, hipStream_t st) override;
  std::vector<std::string> meta_state() const override;
  void set_meta_state(const std::vector<std::string>& v) override;
  std::unique_ptr<Cache> copy(hipStream_t st) override;
  void read_kv(hipStream_t st, vkv_array* k, vkv_array* v) override;
  std::unique_ptr<Cache> to_unquantized(hipStream_t st);
  vkv_paged_view view() const;
  // make room for `cap` tokens per row (reference growth arithmetic is done
  // by the caller); keeps existing blocks in place.
  void reserve(int64_t B, int64_t H, int64_t D, int64_t cap, int dtype, hipStream_t st);
  int group_, bits_, step_;
  int dtype_ = 2;
  int64_t B_ = 0, H_ = 0, D_ = 0, cap_ = 0;
  int64_t nblk_ = 0;  // blocks per row
  int64_t head_bytes_ = 0, block_bytes_ = 0;
  int64_t codes_bytes_ = 0, sb_bytes_ = 0;
  DevBuf store_;
  DevBuf table_;  // int32 [B][nblk_]
  DevBuf state_buf_[6];
  DevBuf kv_buf_[2];
  // updateQuantized's return value (KVCache.swift:1049-1122): the keys'
  // and values' (wq, scales, biases) in the reference layout, [B][H][cap]
  // rows beside the paged store, brought up to date from the store for the
  // tokens written since the last call (tup_valid_ tokens already match);
  // out receives [B, H, offset, *] views of them.  They move (and are
  // gathered whole once) when the capacity grows, as the reference's arrays
  // are re-created then.
  void tuples(hipStream_t st, vkv_array* out);
  DevBuf tup_[6];
  int64_t tup_B_ = 0, tup_H_ = 0, tup_D_ = 0, tup_cap_ = 0, tup_valid_ = 0;
  int tup_dtype_ = -1;
};

class Pool {
 public:
  explicit Pool(const vkv_pool_params& p);
  vkv_pool_params p;
  int64_t head_bytes = 0, block_bytes = 0, layer_bytes = 0;
  ChunkLayout L{};
  DevBuf mem;
  vkv_paged_view view(int layer, const int32_t* table, int32_t stride, const int32_t* lens,
                      int32_t n, int32_t max_len) const;
  void append(int layer, const vkv_array& k, const vkv_array* v, const int32_t* slots, int64_t n,
              hipStream_t st);
};

ChunkLayout chunk_layout(int bits, int dtype, int block_size, int D, int Dv, int group,
                         bool keys_only);

KVSrc kvsrc_from_view(const vkv_paged_view& v);

// PagedCacheManager (Cache/PagedCacheManager.swift) on host, optionally
// bound to a device pool.
class PrefixManager {
 public:
  PrefixManager(int block_size, int max_blocks, const char* model_key, Pool* pool);
  int32_t allocate();
  void free_block(int32_t b);
  void incref(int32_t b);
  int32_t ref_count(int32_t b);
  int32_t find(const std::string& hash);
  void register_block(int32_t b, const std::string& hash);
  void clear();
  void store(const int64_t* tokens, int64_t n, const char* salt, int n_data,
             const int32_t* src_blocks, hipStream_t st);
  void fetch(const int64_t* tokens, int64_t n, const char* salt, int32_t* blocks, int cap,
             int32_t* n_blocks, int64_t* matched);
  vkv_prefix_stats stats();
  int32_t block_tokens(int32_t b);
  // Copy-on-write before a caller writes into block b (see vkv_prefix_writable).
  int32_t writable(int32_t b, hipStream_t st);
  static std::string block_hash(const std::string* parent, const int64_t* tokens, int64_t n,
                                const std::string* model_key, const std::string* salt);

 private:
  struct Block {
    bool has_hash = false;
    std::string hash;
    std::vector<int64_t> tokens;
    bool has_data = false;
    int32_t ref = 0;
    // free-queue links
    int32_t prev = -1, next = -1;
    bool queued = false;
  };
  void q_append(int32_t b);
  int32_t q_pop_first();
  bool q_remove(int32_t b);
  void reset(int32_t b);
  int32_t alloc_locked();
  void free_locked(int32_t b);
  int32_t partial_prefix(const std::string* parent, const std::vector<int64_t>& chunk,
                         const std::string* salt);
  std::mutex mu_;
  int block_size_, max_blocks_;
  bool has_key_;
  std::string key_;
  Pool* pool_;
  std::vector<Block> blocks_;
  int32_t head_ = -1, tail_ = -1;
  std::unordered_map<std::string, int32_t> map_;
  vkv_prefix_stats stats_{};
};

// Split-K workspace for the attention kernels (one per stream).  It only
// grows; outgrown buffers stay allocated (a captured graph may still use
// them) until workspace_release(st), which frees them all and returns the
// bytes released.  Growth during graph capture on `st` is an error.
float* attention_workspace(hipStream_t st, size_t floats);
// At least n zeroed uint32 counters of the stream, for kernels that count
// arrivals and zero their counters again before they end (zeroed once, on
// the stream, when the buffer is allocated or grown; growth during HIP
// graph capture is refused like the workspace's).
uint32_t* attention_counters(hipStream_t st, size_t n);
size_t workspace_release(hipStream_t st);

// TurboQuantKVCache (TurboQuant/TurboQuantKVCache.swift:70-671), in
// vkv_tq_host.cpp.  Fill phase: float K/V appended as KVCacheSimple would
// return them.  Compressed phase: the encoded records of the prefix
// (sink + middle + tail tokens), decoded once into a unified float buffer
// [decoded prefix | window], new tokens written into the window.
struct TqEncoded;
class TurboQuantCache : public Cache {
 public:
  static constexpr int64_t kWindowStep = 256;      // windowStep (:106)
  static constexpr int64_t kMinimumCompressed = 8;  // minimumCompressedTokens (:79)
  TurboQuantCache(int key_bits, int value_bits, int sink, int residual);
  int kind() const override { return VKV_CACHE_TURBOQUANT; }
  bool trimmable() const override { return true; }
  int64_t trim(int64_t n) override;
  int64_t capacity() const override;
  void update(const vkv_array& k, const vkv_array& v, hipStream_t st, vkv_array* ok,
              vkv_array* ov) override;
  int state(hipStream_t, vkv_array* out) override;
  void set_state(const vkv_array* a, int count, hipStream_t st) override;
  void set_meta_state(const std::vector<std::string>&) override {}  // the setter ignores
  std::unique_ptr<Cache> copy(hipStream_t st) override;
  void read_kv(hipStream_t st, vkv_array* k, vkv_array* v) override;

  static bool has_compressible_middle(int64_t tokens, int64_t sink, int64_t residual,
                                      int64_t minimum);
  static std::unique_ptr<TurboQuantCache> from_simple(Cache& src, int key_bits, int value_bits,
                                                      int sink, int residual, hipStream_t st);
  void compress(const vkv_array& k, const vkv_array& v, int64_t source_offset, hipStream_t st);
  void restore_compressed(const vkv_tq_encoded& k, const vkv_tq_encoded& v, int64_t source_offset,
                          const vkv_array* wk, const vkv_array* wv, hipStream_t st);
  void restore_decoded(const vkv_array& k, const vkv_array& v, int64_t source_offset,
                       hipStream_t st);
  bool window_state(vkv_array* k, vkv_array* v) const;
  void encoded(vkv_tq_encoded* k, vkv_tq_encoded* v) const;

  int key_bits_, value_bits_, sink_, residual_;
  int phase_ = 0;  // 0 fill, 1 compressed
  Dense4 fk_, fv_;
  std::shared_ptr<TqEncoded> ck_, cv_;
  Dense4 uk_, uv_;
  int64_t prefix_ = 0, window_ = 0;

 private:
  void reset();
  void seat(std::shared_ptr<TqEncoded> ek, std::shared_ptr<TqEncoded> ev, hipStream_t st);
  void append_window(const vkv_array& k, const vkv_array& v, hipStream_t st);
};
// CompilableTurboQuantKVCache (BatchEngine/CompilableTurboQuantKVCache.swift:
// 57-294): compressed-phase window writes at the offset held in device
// memory (ctr[0] = offset, ctr[1] = window write position).
class CompilableTurboQuantCache : public TurboQuantCache {
 public:
  CompilableTurboQuantCache(int key_bits, int value_bits, int sink, int residual);
  int kind() const override { return VKV_CACHE_COMPILABLE_TURBOQUANT; }
  void update(const vkv_array& k, const vkv_array& v, hipStream_t st, vkv_array* ok,
              vkv_array* ov) override;
  int make_mask(int n, int window, bool return_array, hipStream_t st, vkv_array* mask) override;
  // innerState (:286-293): unified keys and values, window position, offset
  int inner_state(vkv_array* out);
  // init(from:) (:110-160)
  static std::unique_ptr<CompilableTurboQuantCache> from(TurboQuantCache& src, hipStream_t st);
  DevBuf ctr_;
  hipStream_t last_ = nullptr;

 private:
  void reserve_casts();
  std::map<int, DevBuf> masks_;  // one mask buffer per row count, never moved
  DevBuf cast_k_, cast_v_;       // the update cast to the buffers' dtype (cap tokens)
};
void tq_host_tables(int dim, int bits, int seed, float* signs, float* codebook, float* qjl);

// Runs f under the C ABI's error convention (vkv_capi.cpp): returns 0, or 1
// with the exception's message kept for vkv_last_error().
int guarded_call(const std::function<void()>& f);

}  // namespace vkv

struct vkv_cache_s {
  std::unique_ptr<vkv::Cache> impl;
};
struct vkv_pool_s {
  std::unique_ptr<vkv::Pool> impl;
};
struct vkv_prefix_s {
  std::unique_ptr<vkv::PrefixManager> impl;
};
