// vkv_host.cpp -- the per-layer cache state machines, the paged pool and
// the prefix-cache manager.  Each method cites the reference code whose
// observable behaviour it reproduces (paths relative to the vmlx-swift
// checkout); device work is issued through the launchers in
// vkv_kernels.hip.
#include "vkv_host.h"

#include <string.h>

#include <algorithm>
#include <cstdlib>
#include <map>

#include "sha256.h"

namespace vkv {

// ----------------------------------------------------------------- helpers

void check4(const vkv_array& a, const char* name) {
  if (a.ndim != 4) throw Error(std::string(name) + " must be a 4-D array [B, H, S, D]");
  if (a.strides[3] != 1) throw Error(std::string(name) + " last dim must be contiguous");
  if (a.dtype != VKV_F32 && a.dtype != VKV_F16 && a.dtype != VKV_BF16)
    throw Error(std::string(name) + " must be f32, f16 or bf16");
  if (!a.data && a.shape[0] * a.shape[1] * a.shape[2] * a.shape[3] > 0)
    throw Error(std::string(name) + " has no data");
}

vkv_array Dense4::view(int64_t len) const {
  if (len < 0 || len > cap) throw Error("view of " + std::to_string(len) + " tokens over a buffer of " +
                                        std::to_string(cap));
  vkv_array a{};
  a.data = buf ? buf->get() : nullptr;
  a.dtype = dtype;
  a.ndim = 4;
  a.shape[0] = B;
  a.shape[1] = H;
  a.shape[2] = len;
  a.shape[3] = D;
  a.strides[0] = H * cap * D;
  a.strides[1] = cap * D;
  a.strides[2] = D;
  a.strides[3] = 1;
  return a;
}

Dense4 alloc_dense(int64_t B, int64_t H, int64_t cap, int64_t D, int dtype, bool zero,
                          hipStream_t st) {
  Dense4 d;
  d.dtype = dtype;
  d.B = B;
  d.H = H;
  d.cap = cap;
  d.D = D;
  d.buf = std::make_shared<DevBuf>(static_cast<size_t>(B * H * cap * D) * elem_bytes(dtype));
  if (zero && d.buf->size()) VKV_HIP(hipMemsetAsync(d.buf->get(), 0, d.buf->size(), st));
  return d;
}

// dst[:, :, dt0:dt0+len, :] = src[:, :, st0:st0+len, :]  (src any strided 4-D array)
void copy_tokens(const Dense4& dst, int64_t dt0, const vkv_array& src, int64_t st0,
                        int64_t len, hipStream_t st) {
  if (len <= 0) return;
  const int es = elem_bytes(src.dtype);
  int64_t shape[4] = {src.shape[0], src.shape[1], len, src.shape[3]};
  int64_t sstr[4] = {src.strides[0], src.strides[1], src.strides[2], src.strides[3]};
  int64_t dstr[4] = {dst.H * dst.cap * dst.D, dst.cap * dst.D, dst.D, 1};
  const uint8_t* sp = static_cast<const uint8_t*>(src.data) + st0 * src.strides[2] * es;
  uint8_t* dp = dst.buf->bytes() + dt0 * dst.D * es;
  launch_copy4d(es, sp, shape, sstr, dp, dstr, st);
}

// copy_tokens of K and V (tokens [st0, st0 + len) of each into [dt0, ..)),
// in one launch when they share an element size.
void copy_tokens_kv(const Dense4& dk, const Dense4& dv, int64_t dt0, const vkv_array& k,
                    const vkv_array& v, int64_t st0, int64_t len, hipStream_t st) {
  if (len <= 0) return;
  const int es = elem_bytes(k.dtype);
  if (elem_bytes(v.dtype) != es) {
    copy_tokens(dk, dt0, k, st0, len, st);
    copy_tokens(dv, dt0, v, st0, len, st);
    return;
  }
  auto desc = [&](const Dense4& d, const vkv_array& a) {
    Copy4D c;
    c.src = static_cast<const uint8_t*>(a.data) + st0 * a.strides[2] * es;
    c.dst = d.buf->bytes() + dt0 * d.D * es;
    const int64_t n[4] = {a.shape[0], a.shape[1], len, a.shape[3]};
    const int64_t dd[4] = {d.H * d.cap * d.D, d.cap * d.D, d.D, 1};
    for (int i = 0; i < 4; i++) {
      c.n[i] = n[i];
      c.s[i] = a.strides[i];
      c.d[i] = dd[i];
    }
    return c;
  };
  launch_copy4d_pair(es, desc(dk, k), desc(dv, v), st);
}

void copy_dense(const Dense4& dst, int64_t dt0, const Dense4& src, int64_t st0, int64_t len,
                       hipStream_t st) {
  copy_tokens(dst, dt0, src.view(src.cap), st0, len, st);
}

Dense4 dense_from_array(const vkv_array& a, hipStream_t st) {
  Dense4 d = alloc_dense(a.shape[0], a.shape[1], a.shape[2], a.shape[3], a.dtype, false, st);
  copy_tokens(d, 0, a, 0, a.shape[2], st);
  return d;
}

int Cache::causal_array_mask(int n, int64_t off, int window, hipStream_t st, vkv_array* mask) {
  // createCausalMask (KVCache.swift:314-336): [n, off + n] bool, built on
  // the device on `st` into a buffer that only grows
  const int64_t cols = off + n;
  mask_buf_.ensure(static_cast<size_t>(std::max<int64_t>(1, n * cols)));
  launch_causal_mask(n, off, window, mask_buf_.bytes(), st);
  *mask = vkv_array{};
  mask->data = mask_buf_.get();
  mask->dtype = VKV_BOOL;
  mask->ndim = 2;
  mask->shape[0] = n;
  mask->shape[1] = cols;
  mask->strides[0] = cols;
  mask->strides[1] = 1;
  return VKV_MASK_ARRAY;
}

// BaseKVCache.makeMask (KVCache.swift:287-311)
int Cache::make_mask(int n, int window, bool return_array, hipStream_t st, vkv_array* mask) {
  if (n == 1) return VKV_MASK_NONE;
  if (offset > 0 || return_array || (window > 0 && n > window))
    return causal_array_mask(n, offset, window, st, mask);
  return VKV_MASK_CAUSAL;
}

void Cache::write_tokens(const Dense4& dk, const Dense4& dv, int64_t dt0, const vkv_array& k,
                         const vkv_array& v, int64_t len, hipStream_t st) {
  if (defer_token && len == 1) {
    pending.set = true;
    pending.dk = &dk;
    pending.dv = &dv;
    pending.pos = dt0;
    pending.k = k;
    pending.v = v;
    return;
  }
  copy_tokens_kv(dk, dv, dt0, k, v, 0, len, st);
}

void Cache::flush_pending(hipStream_t st) {
  if (!pending.set) return;
  pending.set = false;
  copy_tokens_kv(*pending.dk, *pending.dv, pending.pos, pending.k, pending.v, 0, 1, st);
}

// BaseKVCache.metaState setter (KVCache.swift:268-276)
void Cache::set_meta_state(const std::vector<std::string>& v) {
  if (!(v.size() == 1 && v[0].empty()))
    throw Error("This cache has no meta_state but a meta_state was set.");
}

std::unique_ptr<Cache> make_cache(const vkv_cache_params& p) {
  const int step = p.step > 0 ? p.step : 256;
  switch (p.kind) {
    case VKV_CACHE_SIMPLE: return std::make_unique<SimpleCache>(step);
    case VKV_CACHE_ROTATING:
      if (p.max_size <= 0) throw Error("RotatingKVCache requires maxSize > 0");
      if (p.keep < 0 || p.keep >= p.max_size) throw Error("keep must be in [0, maxSize)");
      return std::make_unique<RotatingCache>(p.max_size, p.keep, step);
    case VKV_CACHE_QUANTIZED: {
      const int group = p.group_size > 0 ? p.group_size : 64;
      const int bits = p.bits > 0 ? p.bits : 8;
      if (bits != 4 && bits != 8) throw Error("QuantizedKVCache bits must be 4 or 8");
      if (group != 32 && group != 64 && group != 128) throw Error("group_size must be 32, 64 or 128");
      return std::make_unique<QuantizedCache>(group, bits, 256);
    }
    case VKV_CACHE_COMPILABLE:
      return std::make_unique<CompilableCache>(p.max_size > 0 ? p.max_size : 4096, step);
    case VKV_CACHE_COMPILABLE_ROTATING:
      if (p.max_size <= 0) throw Error("CompilableRotatingKVCache requires maxSize > 0");
      if (p.keep < 0 || p.keep >= p.max_size) throw Error("keep must be in [0, maxSize)");
      return std::make_unique<CompilableRotatingCache>(p.max_size, p.keep, step);
    case VKV_CACHE_TURBOQUANT:
      return std::make_unique<TurboQuantCache>(p.bits > 0 ? p.bits : 3, p.bits > 0 ? p.bits : 3, 4,
                                               64);
    case VKV_CACHE_COMPILABLE_TURBOQUANT:  // the direct init (:89-108): the parent's fill phase
      return std::make_unique<CompilableTurboQuantCache>(p.bits > 0 ? p.bits : 3,
                                                         p.bits > 0 ? p.bits : 3, 4, 64);
    default: throw Error("unknown cache kind");
  }
}

// ----------------------------------------------------------- KVCacheSimple

// KVCacheSimple.update (KVCache.swift:465-508)
void SimpleCache::update(const vkv_array& k, const vkv_array& v, hipStream_t st, vkv_array* ok,
                         vkv_array* ov) {
  check4(k, "keys");
  check4(v, "values");
  if (k.dtype != v.dtype) throw Error("keys and values must share a dtype");
  const int64_t B = k.shape[0], H = k.shape[1], Sn = k.shape[2], D = k.shape[3], Dv = v.shape[3];
  if (v.shape[0] != B || v.shape[1] != H || v.shape[2] != Sn) throw Error("keys/values shape mismatch");
  if (!k_.empty() && (k_.B != B || k_.H != H || k_.D != D || v_.D != Dv || k_.dtype != k.dtype))
    throw Error("keys do not match the cached [B, H, D] / dtype");
  const int64_t prev = offset;
  const bool reset = k_.empty() || prev + Sn > k_.cap;
  if (reset) {
    const int64_t n_steps = (step_ + Sn - 1) / step_;
    if (!k_.empty()) {
      const int64_t keep = (prev % step_ != 0) ? prev : k_.cap;  // :485-488
      Dense4 nk = alloc_dense(B, H, keep + n_steps * step_, D, k.dtype, true, st);
      Dense4 nv = alloc_dense(B, H, keep + n_steps * step_, Dv, k.dtype, true, st);
      copy_dense(nk, 0, k_, 0, keep, st);
      copy_dense(nv, 0, v_, 0, keep, st);
      k_ = nk;
      v_ = nv;
    } else {
      k_ = alloc_dense(B, H, n_steps * step_, D, k.dtype, true, st);
      v_ = alloc_dense(B, H, n_steps * step_, Dv, k.dtype, true, st);
    }
  }
  offset += Sn;
  write_tokens(k_, v_, prev, k, v, Sn, st);
  *ok = k_.view(offset);
  *ov = v_.view(offset);
}

// KVCacheSimple.trim (KVCache.swift:551-556)
int64_t SimpleCache::trim(int64_t n) {
  const int64_t t = std::min(offset, n);
  offset -= t;
  return t;
}

// KVCacheSimple.state getter (KVCache.swift:527-537)
int SimpleCache::state(hipStream_t, vkv_array* out) {
  if (k_.empty()) return 0;
  // [..<offset] clamps to the buffers' length, as MLX slicing does
  out[0] = k_.view(std::min(offset, k_.cap));
  out[1] = v_.view(std::min(offset, v_.cap));
  return 2;
}

// KVCacheSimple.state setter (KVCache.swift:538-546)
void SimpleCache::set_state(const vkv_array* a, int count, hipStream_t st) {
  if (count != 2) throw Error("KVCacheSimple state must have exactly 2 arrays (keys, values)");
  check4(a[0], "keys");
  check4(a[1], "values");
  k_ = dense_from_array(a[0], st);
  v_ = dense_from_array(a[1], st);
  offset = k_.cap;
}

// KVCacheSimple.copy (KVCache.swift:583-591): a new cache owning copies of
// the trimmed state.
std::unique_ptr<Cache> SimpleCache::copy(hipStream_t st) {
  auto c = std::make_unique<SimpleCache>(step_);
  vkv_array s[2];
  if (state(st, s) == 2) c->set_state(s, 2, st);
  return c;
}

// KVCacheSimple.readKV (KVCache.swift:516-525)
void SimpleCache::read_kv(hipStream_t, vkv_array* k, vkv_array* v) {
  if (k_.empty()) throw Error("nothing cached yet");
  *k = k_.view(std::min(offset, k_.cap));
  *v = v_.view(std::min(offset, v_.cap));
}

// KVCacheSimple.toQuantized (KVCache.swift:561-581)
std::unique_ptr<Cache> SimpleCache::to_quantized(int group, int bits, hipStream_t st) {
  vkv_cache_params p{};
  p.kind = VKV_CACHE_QUANTIZED;
  p.group_size = group;
  p.bits = bits;
  auto base = make_cache(p);
  auto* q = static_cast<QuantizedCache*>(base.get());
  q->offset = offset;
  if (!k_.empty() && offset > 0) {
    q->reserve(k_.B, k_.H, k_.D, offset, k_.dtype, st);
    if (v_.D != k_.D) throw Error("toQuantized needs equal key and value head dims");
    if (offset > k_.cap) throw Error("toQuantized: offset is past the cached tokens");
    vkv_array kv[2] = {k_.view(offset), v_.view(offset)};
    for (int which = 0; which < 2; which++) {
      const vkv_array& a = kv[which];
      RowSrc src{a.data, a.shape[0], a.shape[2], a.shape[1], a.strides[0], a.strides[2], a.strides[1]};
      ChunkLayout L = chunk_layout(bits, a.dtype, QuantizedCache::kBlock, static_cast<int>(q->D_),
                                   static_cast<int>(q->D_), group, false);
      RowDst dst = affine_dst(q->store_.bytes(), q->block_bytes_, q->head_bytes_,
                              QuantizedCache::kBlock, L, which, static_cast<int>(q->D_) / group, false);
      dst.table = static_cast<const int32_t*>(q->table_.get());
      dst.table_stride = static_cast<int32_t>(q->nblk_);
      dst.seq_S = static_cast<int32_t>(offset);
      dst.start = 0;
      launch_quantize_rows(a.dtype, bits, group, 1, src, dst, a.shape[0] * a.shape[1] * a.shape[2],
                           static_cast<int>(a.shape[3]), st);
    }
  }
  return base;
}

// --------------------------------------------------------- RotatingKVCache

// RotatingKVCache.trim(trimSize:_:append:) (KVCache.swift:626-640)
Dense4 RotatingCache::trim_cat(int64_t trim_size, const Dense4& a, const vkv_array* append,
                               hipStream_t st) const {
  int64_t len = 0;
  if (trim_size > 0) len = std::min(keep_, a.cap) + std::max<int64_t>(0, a.cap - (trim_size + keep_));
  else len = a.cap;
  const int64_t app = append ? append->shape[2] : 0;
  Dense4 out = alloc_dense(a.B, a.H, len + app, a.D, a.dtype, false, st);
  if (trim_size > 0) {
    const int64_t k0 = std::min(keep_, a.cap);
    copy_dense(out, 0, a, 0, k0, st);
    copy_dense(out, k0, a, trim_size + keep_, len - k0, st);
  } else {
    copy_dense(out, 0, a, 0, a.cap, st);
  }
  if (append) copy_tokens(out, len, *append, 0, app, st);
  return out;
}

// RotatingKVCache.temporalOrder (KVCache.swift:642-656)
Dense4 RotatingCache::temporal_order(const Dense4& a, hipStream_t st) const {
  if (idx_ == a.cap) return a;
  if (idx_ < offset) {
    Dense4 out = alloc_dense(a.B, a.H, a.cap, a.D, a.dtype, false, st);
    const int64_t k0 = std::min(keep_, a.cap);
    copy_dense(out, 0, a, 0, k0, st);
    copy_dense(out, k0, a, idx_, a.cap - idx_, st);
    copy_dense(out, k0 + (a.cap - idx_), a, keep_, idx_ - keep_, st);
    return out;
  }
  Dense4 out = alloc_dense(a.B, a.H, idx_, a.D, a.dtype, false, st);
  copy_dense(out, 0, a, 0, idx_, st);
  return out;
}

// RotatingKVCache.updateConcat (KVCache.swift:658-680)
void RotatingCache::update_concat(const vkv_array& k, const vkv_array& v, hipStream_t st) {
  if (k_.empty()) {
    k_ = dense_from_array(k, st);
    v_ = dense_from_array(v, st);
  } else {
    k_ = temporal_order(k_, st);
    v_ = temporal_order(v_, st);
    idx_ = k_.cap;
    const int64_t trim_size = idx_ - max_ + 1;
    k_ = trim_cat(trim_size, k_, &k, st);
    v_ = trim_cat(trim_size, v_, &v, st);
  }
  offset += k.shape[2];
  idx_ = k_.cap;
}

// RotatingKVCache.updateInPlace (KVCache.swift:682-769).  Returns false
// when the write had to be handed to updateConcat (:746-756).
bool RotatingCache::update_in_place(const vkv_array& k, const vkv_array& v, hipStream_t st) {
  const int64_t B = k.shape[0], H = k.shape[1], Sn = k.shape[2], D = k.shape[3], Dv = v.shape[3];
  const int64_t prev = offset;
  const int64_t fill = k_.empty() ? 0 : k_.cap;
  if (k_.empty() || (prev >= fill && fill < max_)) {
    const int64_t new_size = std::min(step_, max_ - fill);
    Dense4 nk = alloc_dense(B, H, fill + new_size, D, k.dtype, true, st);
    Dense4 nv = alloc_dense(B, H, fill + new_size, Dv, k.dtype, true, st);
    if (!k_.empty()) {
      copy_dense(nk, 0, k_, 0, fill, st);
      copy_dense(nv, 0, v_, 0, fill, st);
    }
    k_ = nk;
    v_ = nv;
    idx_ = fill;
  }
  const int64_t trim_size = k_.cap - max_;
  if (trim_size > 0) {
    k_ = trim_cat(trim_size, k_, nullptr, st);
    v_ = trim_cat(trim_size, v_, nullptr, st);
    idx_ = max_;
  }
  if (idx_ == max_) idx_ = keep_;
  if (idx_ + Sn > k_.cap) idx_ = keep_;
  if (idx_ + Sn > k_.cap) {
    update_concat(k, v, st);
    return false;
  }
  write_tokens(k_, v_, idx_, k, v, Sn, st);
  offset += Sn;
  idx_ += Sn;
  return true;
}

// RotatingKVCache.canUpdateInPlace (KVCache.swift:780-789)
bool RotatingCache::can_update_in_place(int64_t Sn) const {
  if (k_.empty()) return true;
  const int64_t capacity = k_.cap;
  const bool grown = offset >= capacity && capacity < max_;
  const int64_t effective = grown ? std::min(capacity + step_, max_) : capacity;
  const int64_t start = idx_ >= effective ? keep_ : idx_;
  return start + Sn <= effective;
}

void RotatingCache::outputs(vkv_array* ok, vkv_array* ov) const {
  const int64_t len = offset < k_.cap ? offset : k_.cap;
  *ok = k_.view(len);
  *ov = v_.view(len);
}

// RotatingKVCache.update (KVCache.swift:791-799); the returned arrays
// follow :671-679 (concat: whole buffer) and :764-768 (in place).
void RotatingCache::update(const vkv_array& k, const vkv_array& v, hipStream_t st, vkv_array* ok,
                           vkv_array* ov) {
  check4(k, "keys");
  check4(v, "values");
  if (!k_.empty() && (k_.B != k.shape[0] || k_.H != k.shape[1] || k_.D != k.shape[3] ||
                      k_.dtype != k.dtype))
    throw Error("keys do not match the cached [B, H, D] / dtype");
  bool concat = true;
  if (k.shape[2] == 1 && can_update_in_place(1)) {
    concat = !update_in_place(k, v, st);
  } else {
    update_concat(k, v, st);
  }
  if (concat) {
    *ok = k_.view(k_.cap);
    *ov = v_.view(v_.cap);
  } else {
    outputs(ok, ov);
  }
}

// RotatingKVCache.trim (KVCache.swift:860-865)
int64_t RotatingCache::trim(int64_t n) {
  const int64_t t = std::min(offset, n);
  offset -= t;
  idx_ -= t;
  return t;
}

// RotatingKVCache.state (KVCache.swift:801-823)
int RotatingCache::state(hipStream_t, vkv_array* out) {
  if (k_.empty()) return 0;
  outputs(&out[0], &out[1]);
  return 2;
}

void RotatingCache::set_state(const vkv_array* a, int count, hipStream_t st) {
  if (count != 2) throw Error("RotatingKVCache state must have exactly 2 arrays");
  check4(a[0], "keys");
  check4(a[1], "values");
  k_ = dense_from_array(a[0], st);
  v_ = dense_from_array(a[1], st);
}

// RotatingKVCache.metaState (KVCache.swift:824-853)
std::vector<std::string> RotatingCache::meta_state() const {
  return {std::to_string(keep_), std::to_string(max_), std::to_string(step_),
          std::to_string(offset), std::to_string(idx_)};
}

static bool parse_int(const std::string& s, int64_t* out) {
  if (s.empty()) return false;
  char* end = nullptr;
  long long v = strtoll(s.c_str(), &end, 10);
  if (*end != '\0') return false;
  *out = v;
  return true;
}

void RotatingCache::set_meta_state(const std::vector<std::string>& v) {
  if (v.size() != 5) throw Error("RotatingKVCache metaState must have exactly 5 values");
  int64_t keep, step, off, idx, mx;
  if (!parse_int(v[0], &keep) || !parse_int(v[2], &step) || !parse_int(v[3], &off) ||
      !parse_int(v[4], &idx))
    throw Error("Failed to convert metaState values to integers");
  if (v[1] == "None")
    throw Error("RotatingKVCache requires a non-nil maxSize. Cannot load cache with maxSize=None.");
  if (!parse_int(v[1], &mx)) throw Error("Failed to convert maxCacheSize '" + v[1] + "' to integer");
  keep_ = keep;
  max_ = mx;
  step_ = step;
  offset = off;
  idx_ = idx;
}

// RotatingKVCache.copy (KVCache.swift:947-954)
std::unique_ptr<Cache> RotatingCache::copy(hipStream_t st) {
  auto c = std::make_unique<RotatingCache>(max_, keep_, step_);
  vkv_array s[2];
  if (state(st, s) == 2) c->set_state(s, 2, st);
  c->set_meta_state(meta_state());
  return c;
}

// RotatingKVCache.temporallyOrderedKV (KVCache.swift:876-887)
void RotatingCache::read_kv(hipStream_t st, vkv_array* k, vkv_array* v) {
  if (k_.empty()) throw Error("nothing cached yet");
  ordered_k_ = temporal_order(k_, st);
  ordered_v_ = temporal_order(v_, st);
  const int64_t len = offset < ordered_k_.cap ? offset : ordered_k_.cap;
  *k = ordered_k_.view(len);
  *v = ordered_v_.view(len);
}

// RotatingKVCache.makeMask (KVCache.swift:890-927)
int RotatingCache::make_mask(int n, int window, bool return_array, hipStream_t st, vkv_array* mask) {
  if (n > 1) {
    const int64_t actual = window > 0 ? window : max_;
    const int64_t capped = std::min<int64_t>(max_ - 1, offset);
    if (capped + n > actual || return_array)
      return causal_array_mask(n, capped, static_cast<int>(actual), st, mask);
    return VKV_MASK_CAUSAL;
  }
  if (window <= 0) return VKV_MASK_NONE;
  if (offset >= window && max_ > window) {
    int64_t cur = idx_;
    if (cur >= max_) cur = 0;
    const int64_t size = offset < max_ ? offset + 1 : max_;
    // roll(arange(size) >= size - window, shift: cur + 1), built on the device
    mask_buf_.ensure(static_cast<size_t>(size));
    launch_roll_mask(size, window, cur + 1, mask_buf_.bytes(), st);
    *mask = vkv_array{};
    mask->data = mask_buf_.get();
    mask->dtype = VKV_BOOL;
    mask->ndim = 1;
    mask->shape[0] = size;
    mask->strides[0] = 1;
    return VKV_MASK_ARRAY;
  }
  return VKV_MASK_NONE;
}

// ------------------------------------------------------ CompilableKVCache

static DevBuf make_counters() {
  DevBuf c(2 * sizeof(int32_t));
  VKV_HIP(hipMemset(c.get(), 0, c.size()));
  return c;
}

static vkv_array counter_array(const DevBuf& c, int slot) {
  vkv_array a{};
  a.data = static_cast<int32_t*>(c.get()) + slot;
  a.dtype = VKV_I32;
  a.ndim = 1;
  a.shape[0] = 1;
  a.strides[0] = 1;
  return a;
}

static std::pair<int64_t, int64_t> read_counters(const DevBuf& c, hipStream_t last) {
  if (last) VKV_HIP(hipStreamSynchronize(last));
  int32_t h[2];
  VKV_HIP(hipMemcpy(h, c.get(), sizeof(h), hipMemcpyDeviceToHost));
  return {h[0], h[1]};
}

// d[:, :, start + i, :] = a[:, :, i, :] with start the int32 at `start`
// (dynamicSliceUpdate along axis 2, DynamicSlice.swift:50-71)
static void write_at_device_offset(const Dense4& d, const vkv_array& a, const int32_t* start,
                                   hipStream_t st) {
  DynCopy c{};
  c.src = static_cast<const uint8_t*>(a.data);
  c.dst = d.buf->bytes();
  const int64_t dstr[4] = {d.H * d.cap * d.D, d.cap * d.D, d.D, 1};
  for (int i = 0; i < 4; i++) {
    c.sstr[i] = a.strides[i];
    c.dstr[i] = dstr[i];
    c.shape[i] = a.shape[i];
  }
  c.axis = 2;
  c.on_dst = 1;
  c.limit = d.cap;
  c.start = start;
  launch_dyn_copy(elem_bytes(a.dtype), c, st);
}

static void check_kv_pair(const vkv_array& k, const vkv_array& v) {
  check4(k, "keys");
  check4(v, "values");
  if (k.shape[0] != v.shape[0] || k.shape[1] != v.shape[1] || k.shape[2] != v.shape[2] ||
      k.dtype != v.dtype)
    throw Error("keys and values must agree in batch, heads, length and dtype");
}

static void check_fits(const Dense4& d, const vkv_array& a, const char* name) {
  if (d.B != a.shape[0] || d.H != a.shape[1] || d.D != a.shape[3] || d.dtype != a.dtype)
    throw Error(std::string(name) + " do not match the cache's fixed buffers");
}

static int full_mask(std::map<int, DevBuf>& masks, const DevBuf& ctr, int n, int64_t cols, int window,
                     int ring, hipStream_t st, vkv_array* mask) {
  if (n < 1) throw Error("n must be >= 1");
  DevBuf& b = masks[n];
  const size_t need = static_cast<size_t>(n) * cols;
  b.ensure(need);
  launch_offset_mask(static_cast<const int32_t*>(ctr.get()), n, static_cast<int>(cols), window, ring,
                     b.bytes(), st);
  *mask = vkv_array{};
  mask->data = b.get();
  mask->dtype = VKV_BOOL;
  mask->ndim = 2;
  mask->shape[0] = n;
  mask->shape[1] = cols;
  mask->strides[0] = cols;
  mask->strides[1] = 1;
  return VKV_MASK_ARRAY;
}

CompilableCache::CompilableCache(int64_t max_length, int step)
    : max_(max_length), step_(step), ctr_(make_counters()) {}

std::pair<int64_t, int64_t> CompilableCache::counters() const { return read_counters(ctr_, last_); }

void CompilableCache::alloc_buffers(const vkv_array& k, const vkv_array& v, int64_t len,
                                    hipStream_t st) {
  k_ = alloc_dense(k.shape[0], k.shape[1], len, k.shape[3], k.dtype, true, st);
  v_ = alloc_dense(v.shape[0], v.shape[1], len, v.shape[3], v.dtype, true, st);
}

// update(keys:values:) (CompilableKVCache.swift:115-149): allocate zeroed
// [B, H, maxLength, D] buffers on first use, write the new tokens at the
// device offset, advance it on the device, return the whole buffers.
void CompilableCache::update(const vkv_array& k, const vkv_array& v, hipStream_t st, vkv_array* ok,
                             vkv_array* ov) {
  check_kv_pair(k, v);
  if (k_.empty()) {
    alloc_buffers(k, v, max_, st);
  } else {
    check_fits(k_, k, "keys");
    check_fits(v_, v, "values");
  }
  const int64_t S = k.shape[2];
  if (S > max_) throw Error("update is longer than the cache's maxLength");
  int32_t* ctr = static_cast<int32_t*>(ctr_.get());
  write_at_device_offset(k_, k, ctr, st);
  write_at_device_offset(v_, v, ctr, st);
  launch_counter_advance(ctr, static_cast<int>(S), 0, 0, 0, st);
  last_ = st;
  *ok = k_.view(max_);
  *ov = v_.view(max_);
}

// state getter (CompilableKVCache.swift:197-211): the whole buffers when
// full, else [.., ..<offset, ..]
int CompilableCache::state(hipStream_t, vkv_array* out) {
  if (k_.empty()) return 0;
  const int64_t off = std::max<int64_t>(0, std::min<int64_t>(counters().first, k_.cap));
  out[0] = k_.view(off);
  out[1] = v_.view(off);
  return 2;
}

// state setter (CompilableKVCache.swift:212-225): fresh zeroed maxLength
// buffers holding the arrays at [0, len), offset = len
void CompilableCache::set_state(const vkv_array* a, int count, hipStream_t st) {
  if (count != 2) throw Error("CompilableKVCache state must have exactly 2 arrays (keys, values)");
  check_kv_pair(a[0], a[1]);
  const int64_t len = a[0].shape[2];
  if (len > max_) throw Error("state is longer than the cache's maxLength");
  alloc_buffers(a[0], a[1], max_, st);
  copy_tokens(k_, 0, a[0], 0, len, st);
  copy_tokens(v_, 0, a[1], 0, len, st);
  launch_counter_set(static_cast<int32_t*>(ctr_.get()), static_cast<int32_t>(len), 0, st);
  last_ = st;
}

void CompilableCache::init_from(const vkv_array* state, int count, hipStream_t st) {
  if (count < 2) return;  // an empty source: nothing to copy
  for (int i = 0; i < 2; i++)
    if (state[i].dtype != VKV_F32 && state[i].dtype != VKV_F16 && state[i].dtype != VKV_BF16)
      throw Error("CompilableKVCache(from:) needs a cache whose state is float keys and values");
  set_state(state, 2, st);
}

void CompilableCache::set_offset(int64_t v) {
  launch_counter_set(static_cast<int32_t*>(ctr_.get()), static_cast<int32_t>(v), 0, last_);
}

// trim (CompilableKVCache.swift:229-240): moves the device offset back
int64_t CompilableCache::trim(int64_t n) {
  const int64_t cur = counters().first;
  const int64_t t = std::min(cur, n);
  launch_counter_set(static_cast<int32_t*>(ctr_.get()), static_cast<int32_t>(cur - t), 0, last_);
  return t;
}

// copy (CompilableKVCache.swift:242-257): independent buffers and counter
std::unique_ptr<Cache> CompilableCache::copy(hipStream_t st) {
  if (last_ && last_ != st) VKV_HIP(hipStreamSynchronize(last_));
  auto c = std::make_unique<CompilableCache>(max_, static_cast<int>(step_));
  if (!k_.empty()) {
    c->k_ = alloc_dense(k_.B, k_.H, k_.cap, k_.D, k_.dtype, false, st);
    c->v_ = alloc_dense(v_.B, v_.H, v_.cap, v_.D, v_.dtype, false, st);
    copy_dense(c->k_, 0, k_, 0, k_.cap, st);
    copy_dense(c->v_, 0, v_, 0, v_.cap, st);
  }
  VKV_HIP(hipMemcpyAsync(c->ctr_.get(), ctr_.get(), ctr_.size(), hipMemcpyDeviceToDevice, st));
  c->last_ = st;
  return c;
}

void CompilableCache::read_kv(hipStream_t st, vkv_array* k, vkv_array* v) {
  vkv_array s[2];
  if (state(st, s) != 2) throw Error("nothing cached yet");
  *k = s[0];
  *v = s[1];
}

// makeMask (CompilableKVCache.swift:167-193): always an array mask over the
// whole buffer, built on the device from the offset
int CompilableCache::make_mask(int n, int window, bool, hipStream_t st, vkv_array* mask) {
  return full_mask(masks_, ctr_, n, max_, window, 0, st, mask);
}

int CompilableCache::inner_state(vkv_array* out) {
  int c = 0;
  if (!k_.empty()) {
    out[c++] = k_.view(k_.cap);
    out[c++] = v_.view(v_.cap);
  }
  out[c++] = counter_array(ctr_, 0);
  return c;
}

// ------------------------------------------ CompilableTurboQuantKVCache

CompilableTurboQuantCache::CompilableTurboQuantCache(int key_bits, int value_bits, int sink,
                                                     int residual)
    : TurboQuantCache(key_bits, value_bits, sink, residual), ctr_(make_counters()) {}

// init(from:) (CompilableTurboQuantKVCache.swift:110-160): restoreCompressed
// from the source's records and window, then the counters from its window
// position and offset
std::unique_ptr<CompilableTurboQuantCache> CompilableTurboQuantCache::from(TurboQuantCache& src,
                                                                           hipStream_t st) {
  if (src.phase_ != 1 || !src.ck_ || !src.cv_)
    throw Error("CompilableTurboQuantKVCache(from:) requires a cache in the compressed phase");
  auto c = std::make_unique<CompilableTurboQuantCache>(src.key_bits_, src.value_bits_, src.sink_,
                                                       src.residual_);
  vkv_tq_encoded ek{}, ev{};
  src.encoded(&ek, &ev);
  vkv_array wk{}, wv{};
  const bool window = src.window_state(&wk, &wv);
  c->restore_compressed(ek, ev, src.offset, window ? &wk : nullptr, window ? &wv : nullptr, st);
  launch_counter_set(static_cast<int32_t*>(c->ctr_.get()), static_cast<int32_t>(c->offset),
                     static_cast<int32_t>(c->window_), st);
  c->last_ = st;
  c->reserve_casts();
  return c;
}

// The cast scratch of a compressed-phase update (tokens of another dtype
// than the unified buffers'), sized once for the longest update the buffers
// take, when the buffers are made: an update under HIP-graph capture then
// neither allocates nor frees, and a captured graph's scratch address stays
// valid.
void CompilableTurboQuantCache::reserve_casts() {
  if (phase_ != 1 || uk_.empty()) return;
  cast_k_.ensure(static_cast<size_t>(uk_.B * uk_.H * uk_.cap * uk_.D) * elem_bytes(uk_.dtype));
  cast_v_.ensure(static_cast<size_t>(uv_.B * uv_.H * uv_.cap * uv_.D) * elem_bytes(uv_.dtype));
}

// update (:168-224): the fill phase is the parent's; compressed, the new
// tokens go to the unified buffers at the device offset (dynamicSliceUpdate:
// cast to the buffers' dtype, start clamped so they fit), both counters and
// the host offset and window position advance, and the whole buffers return
void CompilableTurboQuantCache::update(const vkv_array& k, const vkv_array& v, hipStream_t st,
                                       vkv_array* ok, vkv_array* ov) {
  if (phase_ != 1 || uk_.empty()) {
    TurboQuantCache::update(k, v, st, ok, ov);
    reserve_casts();  // the update that promotes the cache makes its buffers
    return;
  }
  check_kv_pair(k, v);
  if (k.shape[0] != uk_.B || k.shape[1] != uk_.H || k.shape[3] != uk_.D || v.shape[3] != uv_.D)
    throw Error("keys and values do not match the cache's unified buffers");
  const int64_t S = k.shape[2];
  if (S > uk_.cap) throw Error("update is longer than the unified buffers");
  int32_t* ctr = static_cast<int32_t*>(ctr_.get());
  if (k.dtype != uk_.dtype || v.dtype != uv_.dtype) {
    // buffers restored another way than from() or a promotion get their
    // cast scratch here, outside a capture (a no-op once it exists)
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    VKV_HIP(hipStreamIsCapturing(st, &cs));
    if (cs == hipStreamCaptureStatusNone) reserve_casts();
  }
  auto put = [&](const Dense4& d, const vkv_array& a, DevBuf& tmp) {
    if (a.dtype == d.dtype) {
      write_at_device_offset(d, a, ctr, st);
      return;
    }
    const int64_t shape[4] = {a.shape[0], a.shape[1], S, a.shape[3]};
    const int64_t dstr[4] = {a.shape[1] * S * a.shape[3], S * a.shape[3], a.shape[3], 1};
    // S <= cap, so the scratch reserved with the buffers holds it
    if (static_cast<size_t>(shape[0] * dstr[0]) * elem_bytes(d.dtype) > tmp.size())
      throw Error("the cast scratch does not hold the update (run one update before capturing)");
    launch_cast4d(a.data, a.dtype, shape, a.strides, tmp.get(), d.dtype, dstr, st);
    vkv_array c{};
    c.data = tmp.get();
    c.dtype = d.dtype;
    c.ndim = 4;
    for (int i = 0; i < 4; i++) {
      c.shape[i] = shape[i];
      c.strides[i] = dstr[i];
    }
    write_at_device_offset(d, c, ctr, st);
  };
  put(uk_, k, cast_k_);
  put(uv_, v, cast_v_);
  launch_counter_advance_both(ctr, static_cast<int>(S), st);
  last_ = st;
  offset += S;
  window_ += S;
  *ok = uk_.view(uk_.cap);
  *ov = uv_.view(uv_.cap);
}

// makeMask (:226-284): an array mask [n, buffer length] from the device
// offset, row i seeing positions <= offset + i (within the window if given)
int CompilableTurboQuantCache::make_mask(int n, int window, bool return_array, hipStream_t st,
                                         vkv_array* mask) {
  if (phase_ != 1 || uk_.empty()) return TurboQuantCache::make_mask(n, window, return_array, st, mask);
  return full_mask(masks_, ctr_, n, uk_.cap, window, 0, st, mask);
}

int CompilableTurboQuantCache::inner_state(vkv_array* out) {
  int c = 0;
  if (!uk_.empty()) {
    out[c++] = uk_.view(uk_.cap);
    out[c++] = uv_.view(uv_.cap);
  }
  out[c++] = counter_array(ctr_, 1);
  out[c++] = counter_array(ctr_, 0);
  return c;
}

// --------------------------------------------- CompilableRotatingKVCache

CompilableRotatingCache::CompilableRotatingCache(int max_size, int keep, int step)
    : RotatingCache(max_size, keep, step), ctr_(make_counters()) {}

void CompilableRotatingCache::pull() const {
  auto* self = const_cast<CompilableRotatingCache*>(this);
  const auto c = read_counters(ctr_, last_);
  self->offset = c.first;
  self->idx_ = c.second;
}

void CompilableRotatingCache::push(hipStream_t st) {
  launch_counter_set(static_cast<int32_t*>(ctr_.get()), static_cast<int32_t>(offset),
                     static_cast<int32_t>(idx_), st);
  last_ = st;
}

int64_t CompilableRotatingCache::current_offset() {
  pull();
  return offset;
}

void CompilableRotatingCache::set_offset(int64_t v) {
  pull();
  offset = v;
  push(last_);
}

bool CompilableRotatingCache::trimmable() const {
  pull();
  return offset < max_;
}

int64_t CompilableRotatingCache::trim(int64_t n) {
  pull();
  const int64_t t = RotatingCache::trim(n);
  push(last_);
  return t;
}

// update (CompilableRotatingKVCache.swift:157-207): allocate the buffers at
// maxSize on first use, write at the device ring index, advance the index
// with the ring wrap and the offset on the device, return the whole buffers.
void CompilableRotatingCache::update(const vkv_array& k, const vkv_array& v, hipStream_t st,
                                     vkv_array* ok, vkv_array* ov) {
  check_kv_pair(k, v);
  if (k_.empty()) {
    k_ = alloc_dense(k.shape[0], k.shape[1], max_, k.shape[3], k.dtype, true, st);
    v_ = alloc_dense(v.shape[0], v.shape[1], max_, v.shape[3], v.dtype, true, st);
  } else {
    check_fits(k_, k, "keys");
    check_fits(v_, v, "values");
  }
  const int64_t S = k.shape[2];
  if (S > k_.cap) throw Error("update is longer than the ring");
  int32_t* ctr = static_cast<int32_t*>(ctr_.get());
  write_at_device_offset(k_, k, ctr + 1, st);
  write_at_device_offset(v_, v, ctr + 1, st);
  launch_counter_advance(ctr, static_cast<int>(S), 1, static_cast<int>(max_), static_cast<int>(keep_),
                         st);
  last_ = st;
  *ok = k_.view(k_.cap);
  *ov = v_.view(v_.cap);
}

int CompilableRotatingCache::state(hipStream_t st, vkv_array* out) {
  pull();
  return RotatingCache::state(st, out);
}

// state setter: the arrays become the buffers (RotatingKVCache.swift
// :813-822), extended with zeros to maxSize so that device-offset writes
// stay in place (the promotion of CompilableRotatingKVCache.swift:113-140)
void CompilableRotatingCache::set_state(const vkv_array* a, int count, hipStream_t st) {
  if (count != 2) throw Error("RotatingKVCache state must have exactly 2 arrays");
  check_kv_pair(a[0], a[1]);
  const int64_t len = a[0].shape[2];
  const int64_t cap = std::max<int64_t>(len, max_);
  k_ = alloc_dense(a[0].shape[0], a[0].shape[1], cap, a[0].shape[3], a[0].dtype, len < cap, st);
  v_ = alloc_dense(a[1].shape[0], a[1].shape[1], cap, a[1].shape[3], a[1].dtype, len < cap, st);
  copy_tokens(k_, 0, a[0], 0, len, st);
  copy_tokens(v_, 0, a[1], 0, len, st);
  last_ = st;
}

std::vector<std::string> CompilableRotatingCache::meta_state() const {
  pull();
  return RotatingCache::meta_state();
}

void CompilableRotatingCache::set_meta_state(const std::vector<std::string>& v) {
  RotatingCache::set_meta_state(v);
  push(last_);
}

std::unique_ptr<Cache> CompilableRotatingCache::copy(hipStream_t st) {
  if (last_ && last_ != st) VKV_HIP(hipStreamSynchronize(last_));
  auto c = std::make_unique<CompilableRotatingCache>(static_cast<int>(max_), static_cast<int>(keep_),
                                                     static_cast<int>(step_));
  if (!k_.empty()) {
    c->k_ = alloc_dense(k_.B, k_.H, k_.cap, k_.D, k_.dtype, false, st);
    c->v_ = alloc_dense(v_.B, v_.H, v_.cap, v_.D, v_.dtype, false, st);
    copy_dense(c->k_, 0, k_, 0, k_.cap, st);
    copy_dense(c->v_, 0, v_, 0, v_.cap, st);
  }
  VKV_HIP(hipMemcpyAsync(c->ctr_.get(), ctr_.get(), ctr_.size(), hipMemcpyDeviceToDevice, st));
  c->last_ = st;
  return c;
}

void CompilableRotatingCache::read_kv(hipStream_t st, vkv_array* k, vkv_array* v) {
  pull();
  RotatingCache::read_kv(st, k, v);
}

// makeMask (CompilableRotatingKVCache.swift:233-260): causal over the whole
// buffer, all true once the ring is full, then the window
int CompilableRotatingCache::make_mask(int n, int window, bool, hipStream_t st, vkv_array* mask) {
  return full_mask(masks_, ctr_, n, max_, window, 1, st, mask);
}

int CompilableRotatingCache::inner_state(vkv_array* out) {
  int c = 0;
  if (!k_.empty()) {
    out[c++] = k_.view(k_.cap);
    out[c++] = v_.view(v_.cap);
  }
  out[c++] = counter_array(ctr_, 1);
  out[c++] = counter_array(ctr_, 0);
  return c;
}

void CompilableRotatingCache::init_from(const RotatingCache& src, hipStream_t st) {
  offset = src.offset;
  idx_ = src.idx_;
  if (!src.k_.empty()) {
    const int64_t cap = std::max<int64_t>(src.k_.cap, max_);
    k_ = alloc_dense(src.k_.B, src.k_.H, cap, src.k_.D, src.k_.dtype, src.k_.cap < cap, st);
    v_ = alloc_dense(src.v_.B, src.v_.H, cap, src.v_.D, src.v_.dtype, src.v_.cap < cap, st);
    copy_dense(k_, 0, src.k_, 0, src.k_.cap, st);
    copy_dense(v_, 0, src.v_, 0, src.v_.cap, st);
  }
  push(st);
}

// -------------------------------------------------------- QuantizedKVCache

ChunkLayout chunk_layout(int bits, int dtype, int block_size, int D, int Dv, int group,
                         bool keys_only) {
  ChunkLayout L{};
  const int es = elem_bytes(dtype);
  if (bits == 0) {
    L.codes = static_cast<int64_t>(block_size) * D * es;
    L.kc = 0;
    L.vc = static_cast<int32_t>(L.codes);
    L.head = L.codes + static_cast<int64_t>(block_size) * Dv * es;
  } else {
    // K codes | V codes | per-token scale/bias (format in vkv_device.h)
    const int G = D / group;
    L.codes = static_cast<int64_t>(block_size) * D * bits / 8;
    L.sb = static_cast<int64_t>(block_size) * (keys_only ? 2 * G : 4 * G) * es;
    L.kc = 0;
    L.vc = keys_only ? 0 : static_cast<int32_t>(L.codes);
    L.sbo = static_cast<int32_t>(keys_only ? L.codes : 2 * L.codes);
    L.head = L.sbo + L.sb;
  }
  L.head = (L.head + 127) / 128 * 128;  // keep every chunk 128-byte aligned
  return L;
}

RowDst affine_dst(uint8_t* base, int64_t block_bytes, int64_t head_bytes, int block_size,
                  const ChunkLayout& L, int which, int G, bool keys_only) {
  RowDst d{};
  d.base = base;
  d.block_bytes = block_bytes;
  d.head_bytes = head_bytes;
  d.block_size = block_size;
  d.is_v = which;
  d.c_off = which ? L.vc : L.kc;
  d.s_off = L.sbo;
  d.G = G;
  d.keys_only = keys_only ? 1 : 0;
  return d;
}

void QuantizedCache::reserve(int64_t B, int64_t H, int64_t D, int64_t cap, int dtype,
                             hipStream_t st) {
  if (D % group_ != 0 || D % 8 != 0) throw Error("head dim must be a multiple of group_size");
  const int64_t need = (cap + kBlock - 1) / kBlock;
  if (!store_.get()) {
    B_ = B;
    H_ = H;
    D_ = D;
    dtype_ = dtype;
    ChunkLayout L = chunk_layout(bits_, dtype, kBlock, static_cast<int>(D), static_cast<int>(D), group_,
                                 false);
    codes_bytes_ = L.codes;
    sb_bytes_ = L.sb;
    head_bytes_ = L.head;
    block_bytes_ = H * L.head;
    nblk_ = 0;
  } else if (B != B_ || H != H_ || D != D_ || dtype != dtype_) {
    throw Error("keys do not match the cached [B, H, D] / dtype");
  }
  if (need > nblk_ || !store_.get()) {
    const int64_t nb = std::max<int64_t>(need, 1);
    DevBuf ns(static_cast<size_t>(nb * B_ * block_bytes_));
    const size_t old = static_cast<size_t>(nblk_ * B_ * block_bytes_);
    if (old) VKV_HIP(hipMemcpyAsync(ns.get(), store_.get(), old, hipMemcpyDeviceToDevice, st));
    if (ns.size() > old) VKV_HIP(hipMemsetAsync(ns.bytes() + old, 0, ns.size() - old, st));
    VKV_HIP(hipStreamSynchronize(st));  // the old store may be read by queued work
    store_ = std::move(ns);
    nblk_ = nb;
    std::vector<int32_t> t(static_cast<size_t>(B_ * nblk_));
    for (int64_t b = 0; b < B_; b++)
      for (int64_t j = 0; j < nblk_; j++) t[b * nblk_ + j] = static_cast<int32_t>(j * B_ + b);
    DevBuf nt(t.size() * sizeof(int32_t));
    VKV_HIP(hipMemcpy(nt.get(), t.data(), t.size() * sizeof(int32_t), hipMemcpyHostToDevice));
    table_ = std::move(nt);
  }
  cap_ = cap;
}

vkv_paged_view QuantizedCache::view() const {
  vkv_paged_view v{};
  v.base = store_.get();
  v.dtype = dtype_;
  v.bits = bits_;
  v.group_size = group_;
  v.n_kv_heads = static_cast<int32_t>(H_);
  v.head_dim = static_cast<int32_t>(D_);
  v.v_head_dim = static_cast<int32_t>(D_);
  v.block_size = kBlock;
  v.flags = 0;
  v.block_bytes = block_bytes_;
  v.head_bytes = head_bytes_;
  v.block_table = static_cast<const int32_t*>(table_.get());
  v.table_stride = static_cast<int32_t>(nblk_);
  v.seq_lens = nullptr;
  v.n_seqs = static_cast<int32_t>(B_);
  v.max_len = static_cast<int32_t>(offset);
  return v;
}

// QuantizedKVCache.updateQuantized (KVCache.swift:1049-1122)
void QuantizedCache::update_quantized(const vkv_array& k, const vkv_array& v, hipStream_t st,
                                      vkv_paged_view* out) {
  const int64_t prev = advance(k, v, st);
  write_tokens(k, v, prev, st);
  *out = view();
}

int64_t QuantizedCache::advance(const vkv_array& k, const vkv_array& v, hipStream_t st) {
  check4(k, "keys");
  check4(v, "values");
  if (k.dtype != v.dtype) throw Error("keys and values must share a dtype");
  if (k.shape[3] != v.shape[3]) throw Error("QuantizedKVCache needs equal key and value head dims");
  const int64_t B = k.shape[0], H = k.shape[1], Sn = k.shape[2], D = k.shape[3];
  const int64_t prev = offset;
  tup_valid_ = std::min(tup_valid_, prev);  // tokens from prev on are rewritten
  if (!store_.get() || prev + Sn > cap_) {
    const int64_t new_steps = ((step_ + Sn - 1) / step_) * step_;
    int64_t cap = new_steps;
    if (store_.get()) cap = ((prev % step_ != 0) ? prev : cap_) + new_steps;  // :1066-1083
    reserve(B, H, D, cap, k.dtype, st);
  } else if (B != B_ || H != H_ || D != D_ || k.dtype != dtype_) {
    throw Error("keys do not match the cached [B, H, D] / dtype");
  }
  offset += Sn;
  return prev;
}

void QuantizedCache::write_tokens(const vkv_array& k, const vkv_array& v, int64_t prev,
                                  hipStream_t st) {
  const int64_t B = k.shape[0], H = k.shape[1], Sn = k.shape[2], D = k.shape[3];
  const vkv_array* arr[2] = {&k, &v};
  ChunkLayout L = chunk_layout(bits_, dtype_, kBlock, static_cast<int>(D_), static_cast<int>(D_), group_,
                               false);
  if (append_affine_supported(bits_, group_, static_cast<int>(D_))) {
    // K and V in one launch; a chunk of whole 8-token groups writes its
    // 4-bit V words with plain stores instead of per-nibble atomics
    const int G = static_cast<int>(D_ / group_);
    RowSrc sk{k.data, B, Sn, H, k.strides[0], k.strides[2], k.strides[1]};
    RowSrc sv{v.data, B, Sn, H, v.strides[0], v.strides[2], v.strides[1]};
    RowDst dk = affine_dst(store_.bytes(), block_bytes_, head_bytes_, kBlock, L, 0, G, false);
    RowDst dv = affine_dst(store_.bytes(), block_bytes_, head_bytes_, kBlock, L, 1, G, false);
    for (RowDst* d : {&dk, &dv}) {
      d->table = static_cast<const int32_t*>(table_.get());
      d->table_stride = static_cast<int32_t>(nblk_);
      d->seq_S = static_cast<int32_t>(Sn);
      d->start = static_cast<int32_t>(prev);
    }
    launch_append_affine(dtype_, bits_, group_, sk, sv, dk, dv, B * Sn, static_cast<int>(H),
                         static_cast<int>(D), true, st);
    return;
  }
  for (int which = 0; which < 2; which++) {
    const vkv_array& a = *arr[which];
    RowSrc src{a.data, a.shape[0], a.shape[2], a.shape[1], a.strides[0], a.strides[2], a.strides[1]};
    RowDst dst = affine_dst(store_.bytes(), block_bytes_, head_bytes_, kBlock, L, which,
                            static_cast<int>(D_ / group_), false);
    dst.table = static_cast<const int32_t*>(table_.get());
    dst.table_stride = static_cast<int32_t>(nblk_);
    dst.seq_S = static_cast<int32_t>(Sn);
    dst.start = static_cast<int32_t>(prev);
    launch_quantize_rows(a.dtype, bits_, group_, 1, src, dst, B * H * Sn, static_cast<int>(D), st);
  }
}

int64_t QuantizedCache::trim(int64_t n) {
  const int64_t t = std::min(offset, n);
  offset -= t;
  return t;
}

// QuantizedKVCache.state getter (KVCache.swift:1133-1151): the tuples in
// the reference layout, trimmed to offset.
int QuantizedCache::state(hipStream_t st, vkv_array* out) {
  if (!store_.get()) return 0;
  const int64_t T = std::min(offset, cap_);
  const int64_t W = D_ * bits_ / 32, G = D_ / group_;
  const int es = elem_bytes(dtype_);
  vkv_paged_view vw = view();
  vw.max_len = static_cast<int32_t>(T);
  KVSrc kv = kvsrc_from_view(vw);
  for (int which = 0; which < 2; which++) {
    DevBuf& c = state_buf_[3 * which];
    DevBuf& s = state_buf_[3 * which + 1];
    DevBuf& b = state_buf_[3 * which + 2];
    c.ensure(static_cast<size_t>(std::max<int64_t>(1, B_ * H_ * T * W) * 4));
    s.ensure(static_cast<size_t>(std::max<int64_t>(1, B_ * H_ * T * G) * es));
    b.ensure(static_cast<size_t>(std::max<int64_t>(1, B_ * H_ * T * G) * es));
    GatherArgs g{};
    g.kv = kv;
    g.n_seqs = static_cast<int32_t>(B_);
    g.H = static_cast<int32_t>(H_);
    g.T = static_cast<int32_t>(T);
    g.D = static_cast<int32_t>(D_);
    g.which = which;
    g.bits = bits_;
    g.group = group_;
    g.dtype = dtype_;
    g.out = c.get();
    g.out_s = s.get();
    g.out_b = b.get();
    launch_gather(g, 1, st);
    const int64_t ws[3] = {W, G, G};
    const int dts[3] = {VKV_U32, dtype_, dtype_};
    for (int i = 0; i < 3; i++) {
      vkv_array& a = out[3 * which + i];
      a = vkv_array{};
      a.data = state_buf_[3 * which + i].get();
      a.dtype = dts[i];
      a.ndim = 4;
      a.shape[0] = B_;
      a.shape[1] = H_;
      a.shape[2] = T;
      a.shape[3] = ws[i];
      a.strides[0] = H_ * T * ws[i];
      a.strides[1] = T * ws[i];
      a.strides[2] = ws[i];
      a.strides[3] = 1;
    }
  }
  return 6;
}

// QuantizedKVCache.state setter (KVCache.swift:1152-1166)
void QuantizedCache::set_state(const vkv_array* a, int count, hipStream_t st) {
  if (count == 4) throw Error("affine QuantizedKVCache state needs biases (6 arrays)");
  if (count != 6)
    throw Error("QuantizedKVCache state must have exactly 6 or 4 arrays (3/2 for keys, 3/2 for values)");
  for (int i = 0; i < 6; i++) {
    if (a[i].ndim != 4) throw Error("quantized state arrays must be 4-D");
    const int64_t* sh = a[i].shape;
    const int64_t* s = a[i].strides;
    if (s[3] != 1 || s[2] != sh[3] || s[1] != sh[2] * sh[3] || s[0] != sh[1] * sh[2] * sh[3])
      throw Error("quantized state arrays must be contiguous");
  }
  const int64_t B = a[0].shape[0], H = a[0].shape[1], T = a[0].shape[2];
  const int64_t D = a[0].shape[3] * 32 / bits_;
  const int dtype = a[1].dtype;
  tup_valid_ = 0;
  store_.release();
  table_.release();
  nblk_ = 0;
  reserve(B, H, D, T, dtype, st);
  ChunkLayout L = chunk_layout(bits_, dtype_, kBlock, static_cast<int>(D_), static_cast<int>(D_), group_,
                               false);
  for (int which = 0; which < 2; which++) {
    ScatterCodesArgs s{};
    s.wq = static_cast<const uint32_t*>(a[3 * which].data);
    s.scales = a[3 * which + 1].data;
    s.biases = a[3 * which + 2].data;
    s.n_seqs = static_cast<int32_t>(B);
    s.H = static_cast<int32_t>(H);
    s.T = static_cast<int32_t>(T);
    s.D = static_cast<int32_t>(D);
    s.bits = bits_;
    s.group = group_;
    s.dtype = dtype_;
    s.is_v = which;
    s.dst = affine_dst(store_.bytes(), block_bytes_, head_bytes_, kBlock, L, which,
                       static_cast<int>(D_ / group_), false);
    s.dst.table = static_cast<const int32_t*>(table_.get());
    s.dst.table_stride = static_cast<int32_t>(nblk_);
    launch_scatter_codes(s, st);
  }
}

void QuantizedCache::tuples(hipStream_t st, vkv_array* out) {
  if (!store_.get()) throw Error("nothing cached yet");
  const int64_t T = std::min(offset, cap_);
  const int64_t W = D_ * bits_ / 32, G = D_ / group_;
  const int es = elem_bytes(dtype_);
  const int64_t ws[3] = {W, G, G};
  if (tup_B_ != B_ || tup_H_ != H_ || tup_D_ != D_ || tup_cap_ != cap_ || tup_dtype_ != dtype_) {
    const int64_t eb[3] = {4, es, es};
    for (int i = 0; i < 6; i++)
      tup_[i].alloc(static_cast<size_t>(std::max<int64_t>(1, B_ * H_ * cap_ * ws[i % 3]) * eb[i % 3]));
    tup_B_ = B_;
    tup_H_ = H_;
    tup_D_ = D_;
    tup_cap_ = cap_;
    tup_dtype_ = dtype_;
    tup_valid_ = 0;
  }
  const int64_t t0 = std::min(tup_valid_, T);
  if (T > t0) {
    vkv_paged_view vw = view();
    vw.max_len = static_cast<int32_t>(T);
    const KVSrc kv = kvsrc_from_view(vw);
    for (int which = 0; which < 2; which++) {
      GatherArgs g{};
      g.kv = kv;
      g.n_seqs = static_cast<int32_t>(B_);
      g.H = static_cast<int32_t>(H_);
      g.T = static_cast<int32_t>(T - t0);
      g.D = static_cast<int32_t>(D_);
      g.which = which;
      g.bits = bits_;
      g.group = group_;
      g.dtype = dtype_;
      g.t_begin = static_cast<int32_t>(t0);
      g.out_cap = static_cast<int32_t>(cap_);
      g.out_t0 = static_cast<int32_t>(t0);
      g.out = tup_[3 * which].get();
      g.out_s = tup_[3 * which + 1].get();
      g.out_b = tup_[3 * which + 2].get();
      launch_gather(g, 1, st);
    }
  }
  tup_valid_ = T;
  const int dts[3] = {VKV_U32, dtype_, dtype_};
  for (int i = 0; i < 6; i++) {
    vkv_array& a = out[i];
    const int64_t w = ws[i % 3];
    a = vkv_array{};
    a.data = tup_[i].get();
    a.dtype = dts[i % 3];
    a.ndim = 4;
    a.shape[0] = B_;
    a.shape[1] = H_;
    a.shape[2] = T;
    a.shape[3] = w;
    a.strides[0] = H_ * cap_ * w;
    a.strides[1] = cap_ * w;
    a.strides[2] = w;
    a.strides[3] = 1;
  }
}

// QuantizedKVCache.metaState (KVCache.swift:1168-1177)
std::vector<std::string> QuantizedCache::meta_state() const {
  return {std::to_string(step_), std::to_string(offset), std::to_string(group_),
          std::to_string(bits_)};
}

void QuantizedCache::set_meta_state(const std::vector<std::string>& v) {
  if (v.size() != 4) throw Error("QuantizedKVCache metaState must have exactly 4 values");
  int64_t off = 0;
  offset = parse_int(v[1], &off) ? off : 0;
}

// QuantizedKVCache.copy (KVCache.swift:1188-1195)
std::unique_ptr<Cache> QuantizedCache::copy(hipStream_t st) {
  auto c = std::make_unique<QuantizedCache>(group_, bits_, step_);
  vkv_array s[6];
  if (state(st, s) == 6) c->set_state(s, 6, st);
  c->set_meta_state(meta_state());
  return c;
}

void QuantizedCache::read_kv(hipStream_t st, vkv_array* k, vkv_array* v) {
  if (!store_.get()) throw Error("nothing cached yet");
  const int64_t T = std::min(offset, cap_);
  vkv_paged_view vw = view();
  vw.max_len = static_cast<int32_t>(T);
  KVSrc kv = kvsrc_from_view(vw);
  vkv_array* outs[2] = {k, v};
  for (int which = 0; which < 2; which++) {
    kv_buf_[which].ensure(static_cast<size_t>(std::max<int64_t>(1, B_ * H_ * T * D_) * elem_bytes(dtype_)));
    GatherArgs g{};
    g.kv = kv;
    g.n_seqs = static_cast<int32_t>(B_);
    g.H = static_cast<int32_t>(H_);
    g.T = static_cast<int32_t>(T);
    g.D = static_cast<int32_t>(D_);
    g.which = which;
    g.bits = bits_;
    g.group = group_;
    g.dtype = dtype_;
    g.out = kv_buf_[which].get();
    launch_gather(g, 0, st);
    Dense4 d;
    d.dtype = dtype_;
    d.B = B_;
    d.H = H_;
    d.cap = T;
    d.D = D_;
    *outs[which] = d.view(T);
    outs[which]->data = kv_buf_[which].get();
  }
}

// QuantizedKVCache.toUnquantized (KVCache.swift:1199-1220)
std::unique_ptr<Cache> QuantizedCache::to_unquantized(hipStream_t st) {
  auto c = std::make_unique<SimpleCache>(256);
  if (store_.get()) {
    vkv_array kv[2];
    read_kv(st, &kv[0], &kv[1]);
    c->set_state(kv, 2, st);
  }
  c->offset = offset;
  return c;
}

// ------------------------------------------------------------ paged pool

Pool::Pool(const vkv_pool_params& pp) : p(pp) {
  if (p.num_blocks < 2) throw Error("pool needs at least 2 blocks (block 0 is the sentinel)");
  if (p.block_size <= 0 || p.n_layers <= 0 || p.n_kv_heads <= 0 || p.head_dim <= 0)
    throw Error("invalid pool geometry");
  if (p.v_head_dim <= 0) p.v_head_dim = p.head_dim;
  if (p.group_size <= 0) p.group_size = 64;
  const bool keys_only = (p.flags & VKV_VIEW_KEYS_ONLY) != 0;
  if (keys_only && p.bits == 0) throw Error("keys-only pools must be affine quantized");
  if (p.bits != 0) {
    if (p.bits != 4 && p.bits != 8) throw Error("bits must be 0, 4 or 8");
    if (p.head_dim % p.group_size || (!keys_only && p.v_head_dim != p.head_dim))
      throw Error("affine pools need head_dim % group_size == 0 and equal K/V dims");
    if (p.block_size % 32 || p.head_dim % 32)
      throw Error("affine pools need block_size and head_dim multiples of 32");
  }
  if (p.dtype != VKV_F16 && p.dtype != VKV_BF16 && p.dtype != VKV_F32)
    throw Error("pool dtype must be f16, bf16 or f32");
  L = chunk_layout(p.bits, p.dtype, p.block_size, p.head_dim, p.v_head_dim, p.group_size, keys_only);
  head_bytes = L.head;
  block_bytes = head_bytes * p.n_kv_heads;
  layer_bytes = block_bytes * p.num_blocks;
  mem.alloc(static_cast<size_t>(layer_bytes * p.n_layers));
  VKV_HIP(hipMemset(mem.get(), 0, mem.size()));
}

vkv_paged_view Pool::view(int layer, const int32_t* table, int32_t stride, const int32_t* lens,
                          int32_t n, int32_t max_len) const {
  if (layer < 0 || layer >= p.n_layers) throw Error("layer out of range");
  vkv_paged_view v{};
  v.base = mem.bytes() + static_cast<int64_t>(layer) * layer_bytes;
  v.dtype = p.dtype;
  v.bits = p.bits;
  v.group_size = p.group_size;
  v.n_kv_heads = p.n_kv_heads;
  v.head_dim = p.head_dim;
  v.v_head_dim = p.v_head_dim;
  v.block_size = p.block_size;
  v.flags = p.flags;
  v.block_bytes = block_bytes;
  v.head_bytes = head_bytes;
  v.block_table = table;
  v.table_stride = stride;
  v.seq_lens = lens;
  v.n_seqs = n;
  v.max_len = max_len;
  return v;
}

static void check3(const vkv_array& a, int64_t H, int64_t D, int dtype, const char* name) {
  if (a.ndim != 3) throw Error(std::string(name) + " must be [N, Hkv, D]");
  if (a.shape[1] != H || a.shape[2] != D)
    throw Error(std::string(name) + " shape does not match the pool [Hkv, D]");
  if (a.strides[2] != 1) throw Error(std::string(name) + " last dim must be contiguous");
  if (a.dtype != dtype) throw Error(std::string(name) + " dtype must match the pool dtype");
}

void Pool::append(int layer, const vkv_array& k, const vkv_array* v, const int32_t* slots, int64_t n,
                  hipStream_t st) {
  if (layer < 0 || layer >= p.n_layers) throw Error("layer out of range");
  if (!slots && n > 0) throw Error("slot_mapping is required");
  const bool keys_only = (p.flags & VKV_VIEW_KEYS_ONLY) != 0;
  check3(k, p.n_kv_heads, p.head_dim, p.dtype, "keys");
  if (k.shape[0] < n) throw Error("keys hold fewer than n_tokens rows");
  if (!keys_only) {
    if (!v) throw Error("values are required");
    check3(*v, p.n_kv_heads, p.v_head_dim, p.dtype, "values");
    if (v->shape[0] < n) throw Error("values hold fewer than n_tokens rows");
  }
  uint8_t* base = mem.bytes() + static_cast<int64_t>(layer) * layer_bytes;
  if (p.bits != 0 && append_affine_supported(p.bits, p.group_size, p.head_dim) &&
      (keys_only || p.v_head_dim == p.head_dim)) {
    // K and V in one launch
    const int G = p.head_dim / p.group_size;
    RowSrc sk{k.data, 1, n, k.shape[1], 0, k.strides[0], k.strides[1]};
    RowSrc sv = sk;
    if (!keys_only) sv = RowSrc{v->data, 1, n, v->shape[1], 0, v->strides[0], v->strides[1]};
    RowDst dk = affine_dst(base, block_bytes, head_bytes, p.block_size, L, 0, G, keys_only);
    RowDst dv = keys_only ? dk : affine_dst(base, block_bytes, head_bytes, p.block_size, L, 1, G, false);
    dk.slots = slots;
    dv.slots = slots;
    dk.slot_limit = dv.slot_limit = static_cast<int64_t>(p.num_blocks) * p.block_size;
    launch_append_affine(p.dtype, p.bits, p.group_size, sk, sv, dk, dv, n, p.n_kv_heads, p.head_dim,
                         !keys_only, st);
    return;
  }
  const int passes = keys_only ? 1 : 2;
  for (int which = 0; which < passes; which++) {
    const vkv_array& a = which ? *v : k;
    RowSrc src{a.data, 1, n, a.shape[1], 0, a.strides[0], a.strides[1]};
    RowDst dst = affine_dst(base, block_bytes, head_bytes, p.block_size, L, which,
                            p.bits ? p.head_dim / p.group_size : 0, keys_only);
    dst.slots = slots;
    dst.slot_limit = static_cast<int64_t>(p.num_blocks) * p.block_size;
    if (p.bits == 0) {
      launch_copy_rows(p.dtype, 1, src, dst, n * a.shape[1], static_cast<int>(a.shape[2]), st);
    } else {
      launch_quantize_rows(p.dtype, p.bits, p.group_size, 1, src, dst, n * a.shape[1],
                           static_cast<int>(a.shape[2]), st);
    }
  }
}

KVSrc kvsrc_from_view(const vkv_paged_view& v) {
  const bool keys_only = (v.flags & VKV_VIEW_KEYS_ONLY) != 0;
  ChunkLayout L = chunk_layout(v.bits, v.dtype, v.block_size, v.head_dim, v.v_head_dim, v.group_size,
                               keys_only);
  if (L.head != v.head_bytes) throw Error("paged view head_bytes does not match its geometry");
  const uint8_t* base = static_cast<const uint8_t*>(v.base);
  const int es = elem_bytes(v.dtype);
  KVSrc s{};
  const int64_t BB = v.block_bytes, HB = v.head_bytes;
  if (v.bits == 0) {
    s.kc = Comp{base + L.kc, BB, HB, static_cast<int64_t>(v.head_dim) * es};
    s.vc = Comp{base + L.vc, BB, HB, static_cast<int64_t>(v.v_head_dim) * es};
  } else {
    if (v.block_size % 32 || v.head_dim % 32) throw Error("affine views need block_size and head_dim multiples of 32");
    s.qfmt = 1;
    s.base = base;
    s.block_bytes = BB;
    s.head_bytes = HB;
    s.kc_off = L.kc;
    s.vc_off = L.vc;
    s.sb_off = L.sbo;
    s.G = v.head_dim / v.group_size;
    s.keys_only = keys_only ? 1 : 0;
    s.D = v.head_dim;
  }
  s.table = v.block_table;
  s.table_stride = v.table_stride;
  s.block_size = v.block_size;
  s.seq_lens = v.seq_lens;
  s.T = v.max_len;
  return s;
}

// ---------------------------------------------------- prefix-cache manager

// PagedCacheManager.init (PagedCacheManager.swift:80-96)
PrefixManager::PrefixManager(int block_size, int max_blocks, const char* model_key, Pool* pool)
    : block_size_(block_size), max_blocks_(max_blocks), has_key_(model_key != nullptr),
      key_(model_key ? model_key : ""), pool_(pool) {
  if (block_size <= 0 || max_blocks < 1) throw Error("invalid prefix-cache geometry");
  if (pool && (pool->p.block_size != block_size || pool->p.num_blocks < max_blocks))
    throw Error("prefix cache geometry does not fit the pool");
  blocks_.resize(static_cast<size_t>(max_blocks));
  for (int i = 1; i < max_blocks; i++) q_append(i);
  stats_.total_blocks = max_blocks;
  stats_.free_blocks = max_blocks - 1;
}

void PrefixManager::q_append(int32_t b) {  // FreeBlockQueue.append (:46-63)
  Block& x = blocks_[b];
  if (x.queued) return;
  x.queued = true;
  x.prev = tail_;
  x.next = -1;
  if (tail_ >= 0) blocks_[tail_].next = b;
  else head_ = b;
  tail_ = b;
}

bool PrefixManager::q_remove(int32_t b) {  // FreeBlockQueue.remove (:80-86)
  Block& x = blocks_[b];
  if (!x.queued) return false;
  if (x.prev >= 0) blocks_[x.prev].next = x.next;
  else head_ = x.next;
  if (x.next >= 0) blocks_[x.next].prev = x.prev;
  else tail_ = x.prev;
  x.prev = x.next = -1;
  x.queued = false;
  return true;
}

int32_t PrefixManager::q_pop_first() {  // FreeBlockQueue.popFirst (:69-73)
  if (head_ < 0) return -1;
  int32_t b = head_;
  q_remove(b);
  return b;
}

void PrefixManager::reset(int32_t b) {  // CacheBlock.reset (CacheBlock.swift:89-96)
  Block& x = blocks_[b];
  x.has_hash = false;
  x.hash.clear();
  x.tokens.clear();
  x.has_data = false;
  x.ref = 0;
}

// _allocateBlock (PagedCacheManager.swift:116-127)
int32_t PrefixManager::alloc_locked() {
  int32_t b = q_pop_first();
  if (b < 0) return -1;
  Block& x = blocks_[b];
  if (x.has_hash) {
    auto it = map_.find(x.hash);
    if (it != map_.end() && it->second == b) map_.erase(it);
    stats_.evictions += 1;
  }
  reset(b);
  x.ref += 1;
  stats_.allocated_blocks += 1;
  stats_.free_blocks -= 1;
  return b;
}

// _freeBlock (PagedCacheManager.swift:142-156)
void PrefixManager::free_locked(int32_t b) {
  Block& x = blocks_[b];
  const bool was_referenced = x.ref > 0;
  x.ref = std::max(0, x.ref - 1);
  if (x.ref == 0) {
    if (!x.has_hash || !x.has_data || x.tokens.empty()) {
      if (x.has_hash) {
        auto it = map_.find(x.hash);
        if (it != map_.end() && it->second == b) map_.erase(it);
      }
      reset(b);
    }
    q_append(b);
    if (was_referenced) {
      stats_.allocated_blocks -= 1;
      stats_.free_blocks += 1;
    }
  }
}

static void check_block(int32_t b, int max) {
  if (b < 0 || b >= max) throw Error("block id out of range");
}

int32_t PrefixManager::allocate() {
  std::lock_guard<std::mutex> g(mu_);
  return alloc_locked();
}

void PrefixManager::free_block(int32_t b) {
  std::lock_guard<std::mutex> g(mu_);
  check_block(b, max_blocks_);
  free_locked(b);
}

void PrefixManager::incref(int32_t b) {
  std::lock_guard<std::mutex> g(mu_);
  check_block(b, max_blocks_);
  Block& x = blocks_[b];
  if (x.ref == 0) {
    if (q_remove(b)) {
      stats_.allocated_blocks += 1;
      stats_.free_blocks -= 1;
    }
  }
  x.ref += 1;
}

int32_t PrefixManager::ref_count(int32_t b) {
  std::lock_guard<std::mutex> g(mu_);
  check_block(b, max_blocks_);
  return blocks_[b].ref;
}

int32_t PrefixManager::block_tokens(int32_t b) {
  std::lock_guard<std::mutex> g(mu_);
  check_block(b, max_blocks_);
  return blocks_[b].has_hash ? static_cast<int32_t>(blocks_[b].tokens.size()) : -1;
}

// Copy-on-write of a block about to be written (the partially filled last
// block of a fetched prefix, or any block another sequence also holds): a
// block the caller alone references and no cache entry names is returned as
// it is; otherwise a fresh block (from the LRU head, which may evict) gets
// a device copy of every layer of b on `st`, the caller's reference moves
// from b to it (b keeps its cache entry and its other holders), and the
// fresh block is returned, unregistered with refcount 1.  -1 when no block
// is free.  Replaces the copy the reference makes of every restored block
// (CacheHelpers.swift:431-552): here only the block written into is copied.
int32_t PrefixManager::writable(int32_t b, hipStream_t st) {
  std::lock_guard<std::mutex> g(mu_);
  check_block(b, max_blocks_);
  Block& x = blocks_[b];
  if (x.ref < 1) throw Error("copy-on-write needs a block the caller references");
  if (x.ref == 1 && !x.has_hash) return b;
  const int32_t nb = alloc_locked();  // b is referenced, so never on the free queue
  if (nb < 0) return -1;
  if (pool_) {
    const int32_t src = b, dst = nb;
    launch_copy_blocks(pool_->mem.bytes(), pool_->layer_bytes, pool_->p.n_layers,
                       pool_->block_bytes, &src, &dst, 1, st);
  }
  free_locked(b);
  return nb;
}

// findCachedBlock (PagedCacheManager.swift:164-180)
int32_t PrefixManager::find(const std::string& hash) {
  std::lock_guard<std::mutex> g(mu_);
  auto it = map_.find(hash);
  if (it != map_.end()) {
    stats_.cache_hits += 1;
    return it->second;
  }
  stats_.cache_misses += 1;
  return -1;
}

// registerBlock (PagedCacheManager.swift:187-192)
void PrefixManager::register_block(int32_t b, const std::string& hash) {
  std::lock_guard<std::mutex> g(mu_);
  check_block(b, max_blocks_);
  blocks_[b].has_hash = true;
  blocks_[b].hash = hash;
  map_[hash] = b;
}

// clear (PagedCacheManager.swift:195-217)
void PrefixManager::clear() {
  std::lock_guard<std::mutex> g(mu_);
  map_.clear();
  while (q_pop_first() >= 0) {
  }
  for (int i = 0; i < max_blocks_; i++) reset(i);
  for (int i = 1; i < max_blocks_; i++) q_append(i);
  stats_ = vkv_prefix_stats{};
  stats_.total_blocks = max_blocks_;
  stats_.free_blocks = max_blocks_ - 1;
}

// CacheBlock.computeBlockHash (CacheBlock.swift:110-146)
std::string PrefixManager::block_hash(const std::string* parent, const int64_t* tokens, int64_t n,
                                      const std::string* model_key, const std::string* salt) {
  Sha256 h;
  if (model_key) h.update(model_key->data(), model_key->size());
  if (salt) {
    static const char tag[] = "|media:";
    h.update(tag, 7);
    h.update(salt->data(), salt->size());
  }
  if (parent) h.update(parent->data(), parent->size());
  // Swift Int is 64-bit little-endian on every supported host: the raw
  // buffer bytes are the tokens' little-endian encodings.
  for (int64_t i = 0; i < n; i++) {
    uint8_t le[8];
    const uint64_t v = static_cast<uint64_t>(tokens[i]);
    for (int j = 0; j < 8; j++) le[j] = static_cast<uint8_t>(v >> (8 * j));
    h.update(le, 8);
  }
  return h.hex_digest();
}

// BlockHashMap.findLongestPartialPrefix (BlockHashMap.swift:42-70)
int32_t PrefixManager::partial_prefix(const std::string* parent, const std::vector<int64_t>& chunk,
                                      const std::string* salt) {
  int32_t best = -1;
  const std::string* mk = has_key_ ? &key_ : nullptr;
  for (const auto& kv : map_) {
    const int32_t b = kv.second;
    const Block& x = blocks_[b];
    const auto& st = x.tokens;
    if (st.empty() || static_cast<int>(st.size()) >= block_size_ || st.size() >= chunk.size())
      continue;
    if (!std::equal(st.begin(), st.end(), chunk.begin())) continue;
    if (!x.has_hash || x.hash != block_hash(parent, st.data(), static_cast<int64_t>(st.size()), mk, salt))
      continue;
    if (best < 0 || st.size() > blocks_[best].tokens.size() ||
        (st.size() == blocks_[best].tokens.size() && b < best))
      best = b;
  }
  return best;
}

// storeTokenSequence (PagedCacheManager.swift:229-310)
void PrefixManager::store(const int64_t* tokens, int64_t n, const char* salt_c, int n_data,
                          const int32_t* src_blocks, hipStream_t st) {
  std::lock_guard<std::mutex> g(mu_);
  std::string salt_s = salt_c ? salt_c : "";
  const std::string* salt = salt_c ? &salt_s : nullptr;
  const std::string* mk = has_key_ ? &key_ : nullptr;
  std::vector<int32_t> pinned;
  std::vector<int32_t> copy_src, copy_dst;
  std::string parent;
  bool has_parent = false;
  int chunk_index = 0;
  int64_t off = 0;
  while (off < n) {
    const int64_t end = std::min<int64_t>(off + block_size_, n);
    std::vector<int64_t> chunk(tokens + off, tokens + end);
    const std::string hash = block_hash(has_parent ? &parent : nullptr, chunk.data(),
                                        static_cast<int64_t>(chunk.size()), mk, salt);
    auto it = map_.find(hash);
    if (it != map_.end()) {
      const int32_t ex = it->second;
      if (blocks_[ex].ref == 0) {
        q_remove(ex);
        stats_.allocated_blocks += 1;
        stats_.free_blocks -= 1;
      }
      blocks_[ex].ref += 1;
      pinned.push_back(ex);
      parent = hash;
      has_parent = true;
      off = end;
      chunk_index += 1;
      continue;
    }
    if (chunk_index >= n_data) break;
    const int32_t b = alloc_locked();
    if (b < 0) break;
    Block& x = blocks_[b];
    x.tokens = chunk;
    x.has_data = true;
    x.has_hash = true;
    x.hash = hash;
    map_[hash] = b;
    pinned.push_back(b);
    if (pool_ && src_blocks) {
      copy_src.push_back(src_blocks[chunk_index]);
      copy_dst.push_back(b);
    }
    parent = hash;
    has_parent = true;
    off = end;
    chunk_index += 1;
  }
  if (!copy_src.empty()) {
    launch_copy_blocks(pool_->mem.bytes(), pool_->layer_bytes, pool_->p.n_layers, pool_->block_bytes,
                       copy_src.data(), copy_dst.data(), static_cast<int>(copy_src.size()), st);
  }
  for (auto r = pinned.rbegin(); r != pinned.rend(); ++r) free_locked(*r);
}

// fetchPrefix (PagedCacheManager.swift:320-376)
void PrefixManager::fetch(const int64_t* tokens, int64_t n, const char* salt_c, int32_t* out, int cap,
                          int32_t* n_blocks, int64_t* matched) {
  std::lock_guard<std::mutex> g(mu_);
  std::string salt_s = salt_c ? salt_c : "";
  const std::string* salt = salt_c ? &salt_s : nullptr;
  const std::string* mk = has_key_ ? &key_ : nullptr;
  std::vector<int32_t> got;
  std::string parent;
  bool has_parent = false;
  int64_t off = 0;
  while (off < n) {
    const int64_t end = std::min<int64_t>(off + block_size_, n);
    std::vector<int64_t> chunk(tokens + off, tokens + end);
    const std::string hash = block_hash(has_parent ? &parent : nullptr, chunk.data(),
                                        static_cast<int64_t>(chunk.size()), mk, salt);
    if (static_cast<int>(got.size()) >= cap) break;  // caller's buffer is full
    auto it = map_.find(hash);
    const bool exact = it != map_.end();
    int32_t b = exact ? it->second : partial_prefix(has_parent ? &parent : nullptr, chunk, salt);
    if (b < 0) {
      stats_.cache_misses += 1;
      break;
    }
    stats_.cache_hits += 1;
    if (blocks_[b].ref == 0) {
      q_remove(b);
      stats_.allocated_blocks += 1;
      stats_.free_blocks -= 1;
    }
    blocks_[b].ref += 1;
    got.push_back(b);
    parent = blocks_[b].hash;
    has_parent = true;
    off += static_cast<int64_t>(blocks_[b].tokens.size());
    if (!exact) break;
  }
  int64_t m = 0;
  for (int32_t b : got) m += static_cast<int64_t>(blocks_[b].tokens.size());
  *matched = m;
  *n_blocks = static_cast<int32_t>(got.size());
  for (size_t i = 0; i < got.size(); i++) out[i] = got[i];
}

vkv_prefix_stats PrefixManager::stats() {
  std::lock_guard<std::mutex> g(mu_);
  return stats_;
}

// ------------------------------------------------------------ kernel timing

namespace {
struct Timing {
  std::mutex mu;
  bool on = false;
  std::vector<hipEvent_t> pool;                      // idle events
  std::vector<std::pair<hipEvent_t, hipEvent_t>> rec[kTimeKinds];
  hipEvent_t take() {
    if (pool.empty()) {
      hipEvent_t e;
      VKV_HIP(hipEventCreate(&e));
      return e;
    }
    hipEvent_t e = pool.back();
    pool.pop_back();
    return e;
  }
};
Timing& timing() {
  static Timing* t = new Timing();
  return *t;
}
}  // namespace

void timing_enable(bool on) {
  Timing& t = timing();
  std::lock_guard<std::mutex> g(t.mu);
  t.on = on;
}

TimedLaunch timing_prepare(int kind) {
  Timing& t = timing();
  std::lock_guard<std::mutex> g(t.mu);
  TimedLaunch r;
  r.kind = kind;
  if (t.on) {
    r.start = t.take();
    r.stop = t.take();
  }
  return r;
}

void timing_commit(const TimedLaunch& r) {
  if (!r.start) return;
  Timing& t = timing();
  std::lock_guard<std::mutex> g(t.mu);
  t.rec[r.kind].emplace_back(r.start, r.stop);
}

void timing_read(int kind, double* total_ms, int* count) {
  Timing& t = timing();
  std::lock_guard<std::mutex> g(t.mu);
  double sum = 0.0;
  for (auto& pr : t.rec[kind]) {
    VKV_HIP(hipEventSynchronize(pr.second));
    float ms = 0.0f;
    VKV_HIP(hipEventElapsedTime(&ms, pr.first, pr.second));
    sum += ms;
    t.pool.push_back(pr.first);
    t.pool.push_back(pr.second);
  }
  *total_ms = sum;
  *count = static_cast<int>(t.rec[kind].size());
  t.rec[kind].clear();
}

// ------------------------------------------------------------ workspace

namespace {
// Per-stream scratch of the attention launchers.  A HIP graph captured on a
// stream keeps the workspace address it was captured with, so a buffer that
// is outgrown is retired, not freed: it stays allocated until
// vkv_workspace_release() for that stream (or the end of the process).
// Growth inside a capture would record an allocation into the graph, so it
// is refused there.  Keyed by (device, stream): the null stream has the same
// handle on every device.
struct StreamWorkspace {
  DevBuf cur;
  std::vector<DevBuf> retired;
  DevBuf counters;
};
std::mutex& ws_mutex() {
  static std::mutex mu;
  return mu;
}
using WsKey = std::pair<int, hipStream_t>;
std::map<WsKey, StreamWorkspace>& ws_map() {
  static auto* m = new std::map<WsKey, StreamWorkspace>();
  return *m;
}
WsKey ws_key(hipStream_t st) {
  int dev = 0;
  VKV_HIP(hipGetDevice(&dev));
  return {dev, st};
}
}  // namespace

float* attention_workspace(hipStream_t st, size_t floats) {
  std::lock_guard<std::mutex> g(ws_mutex());
  StreamWorkspace& w = ws_map()[ws_key(st)];
  if (w.cur.size() < floats * sizeof(float)) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    VKV_HIP(hipStreamIsCapturing(st, &cs));
    if (cs != hipStreamCaptureStatusNone)
      throw Error("the attention workspace of this stream must grow (to " +
                  std::to_string(floats * sizeof(float)) +
                  " bytes) during HIP graph capture: run the same call once before capturing");
    const size_t want = std::max(floats * sizeof(float), w.cur.size() * 2);
    if (w.cur.size()) w.retired.push_back(std::move(w.cur));
    w.cur.alloc(want);
  }
  return static_cast<float*>(w.cur.get());
}

uint32_t* attention_counters(hipStream_t st, size_t n) {
  std::lock_guard<std::mutex> g(ws_mutex());
  StreamWorkspace& w = ws_map()[ws_key(st)];
  if (w.counters.size() < n * sizeof(uint32_t)) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    VKV_HIP(hipStreamIsCapturing(st, &cs));
    if (cs != hipStreamCaptureStatusNone)
      throw Error("the attention counters of this stream must grow during HIP graph capture: "
                  "run the same call once before capturing");
    const size_t want = std::max(n * sizeof(uint32_t), std::max<size_t>(w.counters.size() * 2, 4096));
    if (w.counters.size()) w.retired.push_back(std::move(w.counters));
    w.counters.alloc(want);
    VKV_HIP(hipMemsetAsync(w.counters.get(), 0, want, st));
  }
  return static_cast<uint32_t*>(w.counters.get());
}

size_t workspace_release(hipStream_t st) {
  std::lock_guard<std::mutex> g(ws_mutex());
  auto it = ws_map().find(ws_key(st));
  if (it == ws_map().end()) return 0;
  size_t n = it->second.cur.size() + it->second.counters.size();
  for (auto& b : it->second.retired) n += b.size();
  ws_map().erase(it);  // hipFree waits for the device
  return n;
}

}  // namespace vkv
