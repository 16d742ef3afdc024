// vkv_tq_host.cpp -- TurboQuantKVCache (TurboQuant/TurboQuantKVCache.swift)
// behind the C ABI, and the codec's host-side tables: the Lloyd-Max
// codebooks (TQCodebook.swift), the rotation signs (TQHadamard.swift:52-62,
// srand48 / drand48) and the QJL matrix (TQQJL.swift: MLXRandom.normal on
// key(seed + 1000), i.e. Threefry-2x32 draws mapped through MLX's f32
// erfinv).  The tables are built once per (dim, bits, seed) on the host, as
// the reference builds its EncoderState, and kept on each device for the
// life of the process.
#include <math.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "vkv_host.h"

// every float expression below rounds as written (no fused multiply-add)
#pragma clang fp contract(off)

namespace vkv {
namespace {

// ----------------------------------------------------------------- tables

// POSIX drand48 (srand48 puts the seed's low 32 bits above 0x330E; each
// draw is X <- (0x5DEECE66D X + 0xB) mod 2^48, returned as X / 2^48).
struct Drand48 {
  uint64_t x;
  explicit Drand48(long seed)
      : x((static_cast<uint64_t>(static_cast<uint32_t>(seed)) << 16) | 0x330Eu) {}
  double next() {
    x = (0x5DEECE66Dull * x + 0xBull) & ((1ull << 48) - 1);
    return ldexp(static_cast<double>(x), -48);
  }
};

// Threefry-2x32 with 20 rounds (Salmon et al., SC'11; Random123 rotation
// constants and key-schedule parity), the generator behind MLX's
// random::bits.
void threefry(uint32_t k0, uint32_t k1, uint32_t c0, uint32_t c1, uint32_t* o0, uint32_t* o1) {
  static const int rot[2][4] = {{13, 15, 26, 6}, {17, 29, 16, 24}};
  const uint32_t ks[3] = {k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
  uint32_t x0 = c0 + ks[0], x1 = c1 + ks[1];
  for (int i = 0; i < 5; ++i) {
    for (int r : rot[i & 1]) {
      x0 += x1;
      x1 = (x1 << r) | (x1 >> (32 - r));
      x1 ^= x0;
    }
    x0 += ks[(i + 1) % 3];
    x1 += ks[(i + 2) % 3] + static_cast<uint32_t>(i + 1);
  }
  *o0 = x0;
  *o1 = x1;
}

// MLX's bits(n words, key): the first half of the words from the first
// output of counters (i, i + half + odd), the second half from the second.
std::vector<uint32_t> mlx_bits(uint64_t seed, int64_t n) {
  const uint32_t k0 = static_cast<uint32_t>(seed >> 32), k1 = static_cast<uint32_t>(seed);
  std::vector<uint32_t> out(n);
  const int64_t half = n / 2, odd = n % 2;
  for (int64_t i = 0; i < half; ++i) {
    uint32_t a, b;
    threefry(k0, k1, static_cast<uint32_t>(i), static_cast<uint32_t>(i + half + odd), &a, &b);
    out[i] = a;
    out[half + odd + i] = b;
  }
  if (odd) {
    uint32_t a, b;
    threefry(k0, k1, static_cast<uint32_t>(half), 0, &a, &b);
    out[half] = a;
  }
  return out;
}

// MLX's single-precision erfinv (mlx-generated/metal/erf.h:43-76,
// N. Juffa's published approximation): t = log(1 - a^2), a polynomial in t
// by fused multiply-adds, times a.
float mlx_erfinv(float a) {
  static const float far[9] = {3.03697567e-10f, 2.93243101e-8f, 1.22150334e-6f,
                               2.84108955e-5f,  3.93552968e-4f, 3.02698812e-3f,
                               4.83185798e-3f,  -2.64646143e-1f, 8.40016484e-1f};
  static const float near[10] = {5.43877832e-9f,  1.43285448e-7f,  1.22774793e-6f,
                                 1.12963626e-7f,  -5.61530760e-5f, -1.47697632e-4f,
                                 2.31468678e-3f,  1.15392581e-2f,  -2.32015476e-1f,
                                 8.86226892e-1f};
  const float t = logf(fmaf(a, 0.0f - a, 1.0f));
  const float* c = fabsf(t) > 6.125f ? far : near;
  const int n = fabsf(t) > 6.125f ? 9 : 10;
  float p = c[0];
  for (int i = 1; i < n; ++i) p = fmaf(p, t, c[i]);
  return a * p;
}

// MLXRandom.normal([dim, dim], key: key(seed)): uniform draws on
// (-1 + ulp, 1) -- word / 2^32 in f32, clamped below 1, times the f32 range
// plus the low end -- through sqrt(2) * erfinv.
std::vector<float> qjl_matrix(int dim, uint64_t seed) {
  const int64_t n = static_cast<int64_t>(dim) * dim;
  const std::vector<uint32_t> w = mlx_bits(seed, n);
  const float lo = nextafterf(-1.0f, 0.0f);
  const float range = 1.0f - lo;
  const float top = nextafterf(1.0f, 0.0f);
  const float s2 = static_cast<float>(sqrt(2.0));
  std::vector<float> out(n);
  for (int64_t i = 0; i < n; ++i) {
    float u = static_cast<float>(w[i]) / 4294967296.0f;
    u = std::min(u, top);
    const float x = range * u;
    out[i] = s2 * mlx_erfinv(x + lo);
  }
  return out;
}

float beta_pdf(float x, int d) {
  const double df = d;
  const double lc = lgamma(df / 2.0) - 0.5 * log(M_PI) - lgamma((df - 1.0) / 2.0);
  const double xd = x;
  const double safe = std::max(1.0 - xd * xd, 1e-30);
  const double e = (df - 3.0) / 2.0 * log(safe);
  return static_cast<float>(exp(lc + e));
}

float trapezoid(const float* y, const float* x, int n) {
  float r = 0.0f;
  for (int i = 0; i + 1 < n; ++i) {
    const float dx = x[i + 1] - x[i], sy = y[i] + y[i + 1];
    const float t = dx * sy;
    r += t / 2.0f;
  }
  return r;
}

// TQCodebook.computeCodebook (TQCodebook.swift:103-160): Lloyd-Max for one
// coordinate of a uniform point on the sphere in R^dim, on a 10000-point
// grid, 200 rounds from levels spread over +-3/sqrt(dim), sorted.
std::vector<float> lloyd_max(int dim, int bits) {
  constexpr int kGrid = 10000;
  const int nc = 1 << bits;
  std::vector<float> grid(kGrid), pdf(kGrid), mx, mp, xm;
  mx.reserve(kGrid);
  mp.reserve(kGrid);
  xm.reserve(kGrid);
  for (int i = 0; i < kGrid; ++i) {
    const float f = 2.0f * static_cast<float>(i);
    grid[i] = -1.0f + f / static_cast<float>(kGrid - 1);
  }
  for (int i = 0; i < kGrid; ++i) pdf[i] = beta_pdf(grid[i], dim);
  const float mass0 = trapezoid(pdf.data(), grid.data(), kGrid);
  if (mass0 > 0)
    for (float& p : pdf) p /= mass0;
  const float support = 3.0f / sqrtf(std::max(static_cast<float>(dim), 1.0f));
  std::vector<float> c(nc), bnd(nc + 1);
  for (int i = 0; i < nc; ++i) {
    const float f = 2.0f * support * static_cast<float>(i);
    c[i] = -support + f / static_cast<float>(std::max(nc - 1, 1));
  }
  for (int it = 0; it < 200; ++it) {
    bnd[0] = -1.0f;
    bnd[nc] = 1.0f;
    for (int i = 0; i + 1 < nc; ++i) bnd[i + 1] = (c[i] + c[i + 1]) / 2.0f;
    for (int i = 0; i < nc; ++i) {
      mx.clear();
      mp.clear();
      for (int j = 0; j < kGrid; ++j)
        if (grid[j] >= bnd[i] && grid[j] < bnd[i + 1]) {
          mx.push_back(grid[j]);
          mp.push_back(pdf[j]);
        }
      if (mx.size() < 2) continue;
      const int m = static_cast<int>(mx.size());
      const float mass = trapezoid(mp.data(), mx.data(), m);
      xm.resize(m);
      for (int j = 0; j < m; ++j) xm[j] = mx[j] * mp[j];
      const float mom = trapezoid(xm.data(), mx.data(), m);
      c[i] = mom / std::max(mass, 1e-10f);
    }
  }
  std::sort(c.begin(), c.end());
  return c;
}

std::vector<float> random_signs(int dim, long seed) {
  Drand48 r(seed);
  std::vector<float> s(dim);
  for (int i = 0; i < dim; ++i) s[i] = r.next() < 0.5 ? -1.0f : 1.0f;
  return s;
}

TqBlocks pow2_blocks(int dim) {
  TqBlocks b{};
  int off = 0;
  while (dim > 0) {
    int p = 1;
    while (p * 2 <= dim) p *= 2;
    VKV_CHECK(b.n < 16, "too many Hadamard blocks");
    b.size[b.n] = p;
    b.off[b.n] = off;
    b.scale[b.n] = 1.0f / sqrtf(static_cast<float>(p));
    ++b.n;
    off += p;
    dim -= p;
  }
  return b;
}

// One EncoderState half (keys or values) on one device.
struct TqTables {
  int dim = 0, bits = 0, seed = 0;
  bool qjl = false;
  TqBlocks blocks{};
  DevBuf signs, codebook, bounds, S, St;
};

std::mutex g_tq_mutex;

const std::vector<float>& codebook_host(int dim, int bits) {
  static std::map<std::pair<int, int>, std::vector<float>> cache;
  auto key = std::make_pair(dim, bits);
  auto it = cache.find(key);
  if (it == cache.end()) it = cache.emplace(key, lloyd_max(dim, bits)).first;
  return it->second;
}

void upload(DevBuf& b, const std::vector<float>& v) {
  b.alloc(v.size() * sizeof(float));
  VKV_HIP(hipMemcpy(b.get(), v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice));
}

// The device tables of (dim, bits, seed) for keys (qjl) or values, built on
// first use on the current device and kept until the process ends.
const TqTables& tables(int dim, int bits, int seed, bool qjl) {
  int dev = 0;
  VKV_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> g(g_tq_mutex);
  static std::map<std::tuple<int, int, int, int, bool>, std::unique_ptr<TqTables>> reg;
  auto key = std::make_tuple(dev, dim, bits, seed, qjl);
  auto it = reg.find(key);
  if (it != reg.end()) return *it->second;
  auto t = std::make_unique<TqTables>();
  t->dim = dim;
  t->bits = bits;
  t->seed = seed;
  t->qjl = qjl;
  t->blocks = pow2_blocks(dim);
  const std::vector<float>& cb = codebook_host(dim, bits);
  std::vector<float> bnd(cb.size() - 1);
  for (size_t i = 0; i + 1 < cb.size(); ++i) bnd[i] = (cb[i] + cb[i + 1]) / 2.0f;
  if (bnd.empty()) bnd.push_back(0.0f);
  upload(t->signs, random_signs(dim, seed));
  upload(t->codebook, cb);
  upload(t->bounds, bnd);
  if (qjl) {
    const std::vector<float> S = qjl_matrix(dim, static_cast<uint64_t>(seed) + 1000);
    std::vector<float> St(S.size());
    for (int i = 0; i < dim; ++i)
      for (int j = 0; j < dim; ++j) St[static_cast<size_t>(i) * dim + j] = S[static_cast<size_t>(j) * dim + i];
    upload(t->S, S);
    upload(t->St, St);
  }
  return *reg.emplace(key, std::move(t)).first->second;
}

int promote(int a, int b) { return a == b ? a : VKV_F32; }

vkv_array flat_u32(const DevBuf& b, int64_t n) {
  vkv_array a{};
  a.data = b.get();
  a.dtype = VKV_U32;
  a.ndim = 1;
  a.shape[0] = n;
  a.strides[0] = 1;
  return a;
}

vkv_array norms_view(const DevBuf& b, int64_t B, int64_t H, int64_t Tc) {
  vkv_array a{};
  a.data = b.get();
  a.dtype = VKV_F16;
  a.ndim = 4;
  a.shape[0] = B;
  a.shape[1] = H;
  a.shape[2] = Tc;
  a.shape[3] = 1;
  a.strides[0] = H * Tc;
  a.strides[1] = Tc;
  a.strides[2] = 1;
  a.strides[3] = 1;
  return a;
}

// Copies tokens [s0, s0 + len) of src into dst at token d0, converting.
void cast_tokens(const Dense4& dst, int64_t d0, const vkv_array& src, int64_t s0, int64_t len,
                 hipStream_t st) {
  if (len <= 0) return;
  if (src.dtype == dst.dtype) {
    copy_tokens(dst, d0, src, s0, len, st);
    return;
  }
  const int64_t shape[4] = {src.shape[0], src.shape[1], len, src.shape[3]};
  const int64_t sstr[4] = {src.strides[0], src.strides[1], src.strides[2], src.strides[3]};
  const int64_t dstr[4] = {dst.H * dst.cap * dst.D, dst.cap * dst.D, dst.D, 1};
  const uint8_t* sp =
      static_cast<const uint8_t*>(src.data) + s0 * src.strides[2] * elem_bytes(src.dtype);
  uint8_t* dp = dst.buf->bytes() + d0 * dst.D * elem_bytes(dst.dtype);
  launch_cast4d(sp, src.dtype, shape, sstr, dp, dst.dtype, dstr, st);
}

int64_t words_for(int64_t n, int bits) {
  const int vpw = 32 / bits;
  return (n + vpw - 1) / vpw;
}

}  // namespace

// EncodedKeys / EncodedValues (TQEncodedData.swift:38-170) in device memory.
struct TqEncoded {
  bool keys = false;
  int64_t B = 0, H = 0, Tc = 0, D = 0;
  int index_bits = 0, seed = 42;
  DevBuf indices, qjl, res_norms, vec_norms;
  Dense4 sink, tail;  // exact leading / trailing tokens (input dtype)
  int64_t n_elems() const { return B * H * Tc * D; }
  int64_t sink_count() const { return sink.empty() ? 0 : sink.cap; }
  int64_t tail_count() const { return tail.empty() ? 0 : tail.cap; }
  int64_t tokens() const { return Tc + sink_count() + tail_count(); }
  int input_dtype() const { return !sink.empty() ? sink.dtype : (!tail.empty() ? tail.dtype : -1); }
  // dtype of the decoded tensor: f16, promoted with the exact tokens' dtype
  int decoded_dtype() const {
    int dt = VKV_F16;
    if (!sink.empty()) dt = promote(sink.dtype, dt);
    if (!tail.empty()) dt = promote(tail.dtype, dt);
    return dt;
  }
  void describe(vkv_tq_encoded* e) const;
};

void TqEncoded::describe(vkv_tq_encoded* e) const {
  *e = vkv_tq_encoded{};
  e->indices = flat_u32(indices, words_for(n_elems(), index_bits));
  if (keys) {
    e->qjl = flat_u32(qjl, words_for(n_elems(), 1));
    e->res_norms = norms_view(res_norms, B, H, Tc);
  }
  e->vec_norms = norms_view(vec_norms, B, H, Tc);
  if (!sink.empty()) e->sink = sink.view(sink.cap);
  if (!tail.empty()) e->tail = tail.view(tail.cap);
  e->shape[0] = static_cast<int32_t>(B);
  e->shape[1] = static_cast<int32_t>(H);
  e->shape[2] = static_cast<int32_t>(Tc);
  e->shape[3] = static_cast<int32_t>(D);
  e->index_bits = index_bits;
  e->seed = seed;
}

namespace {

// TQEncoder.encodeKeys / encodeValues (TQEncoder.swift:135-206, :262-312)
// of x [B, H, T, D]: the leading `sink` and trailing `tail` tokens kept
// exact, the middle encoded.
std::shared_ptr<TqEncoded> encode(const vkv_array& x, bool keys, int bits, int seed, int64_t sink,
                                  int64_t tail, hipStream_t st) {
  const int64_t B = x.shape[0], H = x.shape[1], T = x.shape[2], D = x.shape[3];
  const int64_t pre = std::min<int64_t>(std::max<int64_t>(sink, 0), T);
  const int64_t tl = std::min<int64_t>(std::max<int64_t>(tail, 0), std::max<int64_t>(0, T - pre));
  const int64_t mid = T - pre - tl;
  if (mid <= 0)
    throw Error(keys ? "TurboQuant encodeKeys requires at least one compressible token"
                     : "TurboQuant encodeValues requires at least one compressible token");
  if (D < 2 || D > 256) throw Error("TurboQuant head dims must be in [2, 256]");
  const int ib = keys ? std::max(bits - 1, 1) : bits;
  const TqTables& tb = tables(static_cast<int>(D), ib, seed, keys);
  auto e = std::make_shared<TqEncoded>();
  e->keys = keys;
  e->B = B;
  e->H = H;
  e->Tc = mid;
  e->D = D;
  e->index_bits = ib;
  e->seed = seed;
  const int64_t rows = B * H * mid, n = rows * D;
  e->indices.alloc(words_for(n, ib) * 4);
  e->vec_norms.alloc(rows * 2);
  launch_fill_i32(static_cast<int32_t*>(e->indices.get()), words_for(n, ib), 0, st);
  if (keys) {
    e->qjl.alloc(words_for(n, 1) * 4);
    e->res_norms.alloc(rows * 2);
    launch_fill_i32(static_cast<int32_t*>(e->qjl.get()), words_for(n, 1), 0, st);
  }
  if (pre) {
    e->sink = alloc_dense(B, H, pre, D, x.dtype, false, st);
    copy_tokens(e->sink, 0, x, 0, pre, st);
  }
  if (tl) {
    e->tail = alloc_dense(B, H, tl, D, x.dtype, false, st);
    copy_tokens(e->tail, 0, x, T - tl, tl, st);
  }
  TqEncodeArgs a{};
  a.x = x.data;
  a.dtype = x.dtype;
  a.sb = x.strides[0];
  a.sh = x.strides[1];
  a.st = x.strides[2];
  a.B = static_cast<int32_t>(B);
  a.H = static_cast<int32_t>(H);
  a.Tc = static_cast<int32_t>(mid);
  a.t0 = static_cast<int32_t>(pre);
  a.D = static_cast<int32_t>(D);
  a.signs = static_cast<const float*>(tb.signs.get());
  a.codebook = static_cast<const float*>(tb.codebook.get());
  a.bounds = static_cast<const float*>(tb.bounds.get());
  a.nc = 1 << ib;
  a.bits = ib;
  a.St = keys ? static_cast<const float*>(tb.St.get()) : nullptr;
  a.blocks = tb.blocks;
  a.indices = static_cast<uint32_t*>(e->indices.get());
  a.qjl = keys ? static_cast<uint32_t*>(e->qjl.get()) : nullptr;
  a.vec_norms = static_cast<uint16_t*>(e->vec_norms.get());
  a.res_norms = keys ? static_cast<uint16_t*>(e->res_norms.get()) : nullptr;
  launch_tq_encode(a, st);
  return e;
}

// TQEncoder.decodeKeys / decodeValues (TQEncoder.swift:214-255, :315-345)
// into dst tokens [0, e.tokens()): sink, decoded middle, tail.  The state
// is EncoderState(dim, keyBits: index_bits + 1 | valueBits, seed).
void decode_into(const TqEncoded& e, const Dense4& dst, hipStream_t st) {
  const TqTables& tb = tables(static_cast<int>(e.D), e.index_bits, e.seed, e.keys);
  const int64_t pre = e.sink_count();
  if (pre) cast_tokens(dst, 0, e.sink.view(pre), 0, pre, st);
  TqDecodeArgs a{};
  a.indices = static_cast<const uint32_t*>(e.indices.get());
  a.qjl = e.keys ? static_cast<const uint32_t*>(e.qjl.get()) : nullptr;
  a.vec_norms = static_cast<const uint16_t*>(e.vec_norms.get());
  a.res_norms = e.keys ? static_cast<const uint16_t*>(e.res_norms.get()) : nullptr;
  a.B = static_cast<int32_t>(e.B);
  a.H = static_cast<int32_t>(e.H);
  a.Tc = static_cast<int32_t>(e.Tc);
  a.D = static_cast<int32_t>(e.D);
  a.bits = e.index_bits;
  a.codebook = static_cast<const float*>(tb.codebook.get());
  a.signs = static_cast<const float*>(tb.signs.get());
  a.S = e.keys ? static_cast<const float*>(tb.S.get()) : nullptr;
  a.qs = static_cast<float>(sqrt(M_PI / 2.0)) / static_cast<float>(e.D);
  a.blocks = tb.blocks;
  a.out = dst.buf->get();
  a.out_dtype = dst.dtype;
  a.t0 = static_cast<int32_t>(pre);
  a.osb = dst.H * dst.cap * dst.D;
  a.osh = dst.cap * dst.D;
  a.ost = dst.D;
  launch_tq_decode(a, st);
  const int64_t tl = e.tail_count();
  if (tl) cast_tokens(dst, pre + e.Tc, e.tail.view(tl), 0, tl, st);
}

}  // namespace

// ------------------------------------------------------ TurboQuantKVCache

TurboQuantCache::TurboQuantCache(int key_bits, int value_bits, int sink, int residual)
    : key_bits_(key_bits), value_bits_(value_bits), sink_(sink), residual_(std::max(0, residual)) {
  if (key_bits < 1 || key_bits > 9) throw Error("TurboQuant keyBits must be in [1, 9]");
  if (value_bits < 1 || value_bits > 8) throw Error("TurboQuant valueBits must be in [1, 8]");
}

int64_t TurboQuantCache::capacity() const { return phase_ == 0 ? fk_.cap : uk_.cap; }

// TurboQuantKVCache.hasCompressibleMiddle (:152-162)
bool TurboQuantCache::has_compressible_middle(int64_t tokens, int64_t sink, int64_t residual,
                                              int64_t minimum) {
  const int64_t pre = std::min(std::max<int64_t>(sink, 0), std::max<int64_t>(tokens, 0));
  const int64_t tail = std::min(std::max<int64_t>(residual, 0), std::max<int64_t>(0, tokens - pre));
  return tokens - pre - tail >= minimum;
}

// resetToEmpty (:648-662)
void TurboQuantCache::reset() {
  phase_ = 0;
  fk_ = Dense4{};
  fv_ = Dense4{};
  ck_.reset();
  cv_.reset();
  uk_ = Dense4{};
  uv_ = Dense4{};
  window_ = 0;
  prefix_ = 0;
  offset = 0;
}

// compressFloatKV (:361-412): encode, decode once into [decoded | 256
// window slots], compressed phase at sourceOffset.
void TurboQuantCache::compress(const vkv_array& k, const vkv_array& v, int64_t source_offset,
                               hipStream_t st) {
  auto ek = encode(k, true, key_bits_, 42, sink_, residual_, st);
  auto ev = encode(v, false, value_bits_, 42, sink_, residual_, st);
  seat(ek, ev, st);
  offset = source_offset;
}

// Zeros in tokens [t0, t0 + len) of every (b, h) row of d (the rest of the
// buffer is written by the caller).
static void zero_token_range(const Dense4& d, int64_t t0, int64_t len, hipStream_t st) {
  const int64_t es = elem_bytes(d.dtype);
  launch_zero_runs(d.buf->bytes() + t0 * d.D * es, d.cap * d.D * es, len * d.D * es, d.B * d.H, st);
}

// The decoded prefix plus windowStep zero slots, as restoreCompressed and
// compressFloatKV build it.
void TurboQuantCache::seat(std::shared_ptr<TqEncoded> ek, std::shared_ptr<TqEncoded> ev,
                           hipStream_t st) {
  const int64_t n = ek->tokens();
  Dense4 uk = alloc_dense(ek->B, ek->H, n + kWindowStep, ek->D, ek->decoded_dtype(), false, st);
  Dense4 uv = alloc_dense(ev->B, ev->H, n + kWindowStep, ev->D, ev->decoded_dtype(), false, st);
  zero_token_range(uk, n, kWindowStep, st);
  zero_token_range(uv, n, kWindowStep, st);
  decode_into(*ek, uk, st);
  decode_into(*ev, uv, st);
  reset();
  ck_ = std::move(ek);
  cv_ = std::move(ev);
  uk_ = uk;
  uv_ = uv;
  prefix_ = n;
  window_ = 0;
  phase_ = 1;
  offset = n;
}

void TurboQuantCache::update(const vkv_array& k, const vkv_array& v, hipStream_t st, vkv_array* ok,
                             vkv_array* ov) {
  check4(k, "keys");
  check4(v, "values");
  const int64_t B = k.shape[0], H = k.shape[1], Sn = k.shape[2];
  if (v.shape[0] != B || v.shape[1] != H || v.shape[2] != Sn) throw Error("keys/values shape mismatch");
  if (phase_ == 0) {
    // appendFloat (:432-447): concatenate after the first `offset` tokens
    if (!fk_.empty() && (fk_.B != B || fk_.H != H || fk_.D != k.shape[3] || fv_.D != v.shape[3]))
      throw Error("keys do not match the cached [B, H, D]");
    if (!fk_.empty() && (fk_.dtype != k.dtype || fv_.dtype != v.dtype))
      throw Error("keys/values dtype differs from the cached dtype");
    if (fk_.empty() || offset + Sn > fk_.cap) {
      const int64_t cap = ((offset + Sn + kWindowStep - 1) / kWindowStep) * kWindowStep;
      Dense4 nk = alloc_dense(B, H, cap, k.shape[3], k.dtype, false, st);
      Dense4 nv = alloc_dense(B, H, cap, v.shape[3], v.dtype, false, st);
      if (!fk_.empty()) {
        copy_dense(nk, 0, fk_, 0, offset, st);
        copy_dense(nv, 0, fv_, 0, offset, st);
      }
      fk_ = nk;
      fv_ = nv;
    }
    copy_tokens(fk_, offset, k, 0, Sn, st);
    copy_tokens(fv_, offset, v, 0, Sn, st);
    offset += Sn;
    *ok = fk_.view(offset);
    *ov = fv_.view(offset);
    return;
  }
  append_window(k, v, st);
  *ok = uk_.view(prefix_ + window_);
  *ov = uv_.view(prefix_ + window_);
}

// appendDecodeTokens (:450-488): write at prefix + window; a buffer too
// short is rebuilt as [buffer[..<writePos] | ceil(S / 256) * 256 zero slots],
// the concatenation promoting its dtype with the new tokens'.
void TurboQuantCache::append_window(const vkv_array& k, const vkv_array& v, hipStream_t st) {
  const int64_t B = k.shape[0], H = k.shape[1], Sn = k.shape[2];
  if (uk_.B != B || uk_.H != H || uk_.D != k.shape[3] || uv_.D != v.shape[3])
    throw Error("keys do not match the cached [B, H, D]");
  offset += Sn;
  const int64_t pos = prefix_ + window_;
  if (pos + Sn > uk_.cap) {
    const int64_t steps = std::max<int64_t>(1, (kWindowStep + Sn - 1) / kWindowStep);
    const int kdt = pos > 0 ? promote(uk_.dtype, k.dtype) : k.dtype;
    const int vdt = pos > 0 ? promote(uv_.dtype, v.dtype) : v.dtype;
    Dense4 nk = alloc_dense(B, H, pos + steps * kWindowStep, k.shape[3], kdt, true, st);
    Dense4 nv = alloc_dense(B, H, pos + steps * kWindowStep, v.shape[3], vdt, true, st);
    if (pos > 0) {
      cast_tokens(nk, 0, uk_.view(uk_.cap), 0, pos, st);
      cast_tokens(nv, 0, uv_.view(uv_.cap), 0, pos, st);
    }
    uk_ = nk;
    uv_ = nv;
  }
  cast_tokens(uk_, pos, k, 0, Sn, st);
  cast_tokens(uv_, pos, v, 0, Sn, st);
  window_ += Sn;
}

// state getter (:492-521)
int TurboQuantCache::state(hipStream_t, vkv_array* out) {
  if (phase_ == 0) {
    if (fk_.empty()) return 0;
    out[0] = fk_.view(offset);
    out[1] = fv_.view(offset);
    return 2;
  }
  // MLX slicing clamps [..<total] to the buffers' length: a compiled cache
  // whose counters ran past the unified buffers returns the whole buffers
  const int64_t total = std::min(prefix_ + window_, std::min(uk_.cap, uv_.cap));
  if (uk_.empty() || total <= 0) return 0;
  out[0] = uk_.view(total);
  out[1] = uv_.view(total);
  return 2;
}

// state setter (:522-533): two or more arrays put the cache back in the
// fill phase holding them; fewer empty it.
void TurboQuantCache::set_state(const vkv_array* a, int count, hipStream_t st) {
  if (count >= 2) {
    check4(a[0], "keys");
    check4(a[1], "values");
    Dense4 k = dense_from_array(a[0], st), v = dense_from_array(a[1], st);
    reset();
    fk_ = k;
    fv_ = v;
    offset = a[0].shape[2];
  } else {
    reset();
  }
}

// trim (:563-606)
int64_t TurboQuantCache::trim(int64_t n) {
  const int64_t trimmed = std::min(offset, n);
  if (trimmed <= 0) return 0;
  const int64_t target = offset - trimmed;
  if (target <= 0) {
    reset();
    return trimmed;
  }
  if (phase_ == 0) {
    offset = target;
    return trimmed;
  }
  const int64_t used = prefix_ + window_;
  if (target >= prefix_ && target <= used) {
    window_ = target - prefix_;
    offset = target;
    return trimmed;
  }
  // decode -> truncate -> re-encode (the lossy decoded tokens, as the
  // reference does), on the null stream; checked before anything changes
  if (!has_compressible_middle(target, sink_, residual_, 1))
    throw Error("TurboQuant encodeKeys requires at least one compressible token");
  hipStream_t st = nullptr;
  Dense4 k = uk_, v = uv_;
  compress(k.view(target), v.view(target), target, st);
  return trimmed;
}

std::unique_ptr<Cache> TurboQuantCache::copy(hipStream_t st) {
  auto c = std::make_unique<TurboQuantCache>(key_bits_, value_bits_, sink_, residual_);
  c->offset = offset;
  c->phase_ = phase_;
  c->prefix_ = prefix_;
  c->window_ = window_;
  c->ck_ = ck_;  // the encoded records are immutable
  c->cv_ = cv_;
  auto dup = [&](const Dense4& d) {
    if (d.empty()) return Dense4{};
    Dense4 n = alloc_dense(d.B, d.H, d.cap, d.D, d.dtype, false, st);
    copy_dense(n, 0, d, 0, d.cap, st);
    return n;
  };
  c->fk_ = dup(fk_);
  c->fv_ = dup(fv_);
  c->uk_ = dup(uk_);
  c->uv_ = dup(uv_);
  return c;
}

void TurboQuantCache::read_kv(hipStream_t st, vkv_array* k, vkv_array* v) {
  vkv_array s[2];
  if (state(st, s) < 2) throw Error("the cache is empty");
  *k = s[0];
  *v = s[1];
}

// fromSimpleCache (:326-356): an empty cache unless the source has a
// compressible middle.
std::unique_ptr<TurboQuantCache> TurboQuantCache::from_simple(Cache& src, int key_bits,
                                                              int value_bits, int sink,
                                                              int residual, hipStream_t st) {
  auto c = std::make_unique<TurboQuantCache>(key_bits, value_bits, sink, residual);
  vkv_array s[6];
  const int n = src.state(st, s);
  const int64_t off = src.current_offset();
  if (n != 2 || off <= 0 || !has_compressible_middle(off, sink, c->residual_, kMinimumCompressed))
    return c;
  c->compress(s[0], s[1], off, st);
  return c;
}

// restoreFromDecodedKV (:281-322)
void TurboQuantCache::restore_decoded(const vkv_array& k, const vkv_array& v, int64_t source_offset,
                                      hipStream_t st) {
  check4(k, "keys");
  check4(v, "values");
  if (source_offset <= 0) return;
  const int64_t n = k.shape[2];
  Dense4 uk = alloc_dense(k.shape[0], k.shape[1], n + kWindowStep, k.shape[3], k.dtype, false, st);
  Dense4 uv = alloc_dense(v.shape[0], v.shape[1], n + kWindowStep, v.shape[3], v.dtype, false, st);
  zero_token_range(uk, n, kWindowStep, st);
  zero_token_range(uv, n, kWindowStep, st);
  copy_tokens(uk, 0, k, 0, n, st);
  copy_tokens(uv, 0, v, 0, n, st);
  reset();
  uk_ = uk;
  uv_ = uv;
  prefix_ = n;
  window_ = 0;
  phase_ = 1;
  offset = source_offset;
}

namespace {

// A caller's encoded record, validated and copied into cache storage.
std::shared_ptr<TqEncoded> import_record(const vkv_tq_encoded& r, bool keys, hipStream_t st) {
  auto e = std::make_shared<TqEncoded>();
  e->keys = keys;
  e->B = r.shape[0];
  e->H = r.shape[1];
  e->Tc = r.shape[2];
  e->D = r.shape[3];
  e->index_bits = r.index_bits;
  e->seed = r.seed;
  if (e->B <= 0 || e->H <= 0 || e->Tc <= 0 || e->D < 2 || e->D > 256)
    throw Error("the encoded shape must be [B, H, Tc, D] with D in [2, 256]");
  if (r.index_bits < 1 || r.index_bits > 8) throw Error("index bits must be in [1, 8]");
  const int64_t n = e->n_elems(), rows = e->B * e->H * e->Tc;
  auto words = [&](const vkv_array& a, int bits, const char* what, DevBuf& dst) {
    if (a.ndim != 1 || (a.dtype != VKV_U32 && a.dtype != VKV_I32) || a.strides[0] != 1 || !a.data)
      throw Error(std::string(what) + " must be a contiguous 1-D u32 array");
    if (a.shape[0] < words_for(n, bits))
      throw Error(std::string(what) + " holds fewer words than the encoded shape needs");
    dst.alloc(words_for(n, bits) * 4);
    VKV_HIP(hipMemcpyAsync(dst.get(), a.data, words_for(n, bits) * 4, hipMemcpyDeviceToDevice, st));
  };
  auto norms = [&](const vkv_array& a, const char* what, DevBuf& dst) {
    int64_t cnt = 1;
    for (int i = 0; i < a.ndim; ++i) cnt *= a.shape[i];
    if (a.dtype != VKV_F16 || !a.data || cnt != rows)
      throw Error(std::string(what) + " must hold B * H * Tc f16 norms");
    int64_t expect = 1;
    for (int i = a.ndim - 1; i >= 0; --i) {
      if (a.shape[i] != 1 && a.strides[i] != expect)
        throw Error(std::string(what) + " must be contiguous");
      expect *= a.shape[i];
    }
    dst.alloc(rows * 2);
    VKV_HIP(hipMemcpyAsync(dst.get(), a.data, rows * 2, hipMemcpyDeviceToDevice, st));
  };
  words(r.indices, r.index_bits, "indices", e->indices);
  norms(r.vec_norms, "vector norms", e->vec_norms);
  if (keys) {
    words(r.qjl, 1, "QJL signs", e->qjl);
    norms(r.res_norms, "residual norms", e->res_norms);
  }
  auto exact = [&](const vkv_array& a, const char* what, Dense4& dst) {
    if (a.ndim == 0) return;
    check4(a, what);
    if (a.shape[0] != e->B || a.shape[1] != e->H || a.shape[3] != e->D)
      throw Error(std::string(what) + " must be [B, H, n, D] like the encoded shape");
    if (a.shape[2] > 0) dst = dense_from_array(a, st);
  };
  exact(r.sink, "sink tokens", e->sink);
  exact(r.tail, "tail tokens", e->tail);
  if (!e->sink.empty() && !e->tail.empty() && e->sink.dtype != e->tail.dtype)
    throw Error("sink and tail tokens must share a dtype");
  return e;
}

}  // namespace

// restoreCompressed (:180-252): decode the records; then the window tokens
// appended after the compression, exactly sourceOffset - prefix of them (a
// mismatch empties the cache, as the reference does).
void TurboQuantCache::restore_compressed(const vkv_tq_encoded& rk, const vkv_tq_encoded& rv,
                                         int64_t source_offset, const vkv_array* wk,
                                         const vkv_array* wv, hipStream_t st) {
  if (rk.shape[3] <= 0 || rv.shape[3] <= 0) return;
  auto ek = import_record(rk, true, st);
  auto ev = import_record(rv, false, st);
  if (ek->B != ev->B || ek->H != ev->H || ek->tokens() != ev->tokens())
    throw Error("encoded keys and values must cover the same [B, H] and token count");
  seat(ek, ev, st);
  const int64_t expect = source_offset - prefix_;
  if (expect < 0) {
    reset();
    return;
  }
  if (expect == 0) {
    if (wk || wv) reset();
    return;
  }
  if (!wk || !wv || wk->ndim != 4 || wv->ndim != 4 || wk->shape[2] != expect ||
      wv->shape[2] != expect) {
    reset();
    return;
  }
  append_window(*wk, *wv, st);
}

// serializedWindowState (:254-263): the exact tokens after the encoded
// prefix, when they end at offset.
bool TurboQuantCache::window_state(vkv_array* k, vkv_array* v) const {
  if (phase_ != 1 || window_ <= 0 || uk_.empty()) return false;
  const int64_t end = prefix_ + window_;
  // the window must end at offset and lie inside the unified buffers
  // (:254-258); a compiled cache's counters can run past them
  if (end != offset || uk_.cap < end || uv_.cap < end) return false;
  vkv_array a = uk_.view(end), b = uv_.view(end);
  const int64_t ek = prefix_ * a.strides[2] * elem_bytes(a.dtype);
  const int64_t ev = prefix_ * b.strides[2] * elem_bytes(b.dtype);
  a.data = static_cast<uint8_t*>(a.data) + ek;
  b.data = static_cast<uint8_t*>(b.data) + ev;
  a.shape[2] = window_;
  b.shape[2] = window_;
  *k = a;
  *v = b;
  return true;
}

void TurboQuantCache::encoded(vkv_tq_encoded* k, vkv_tq_encoded* v) const {
  if (!ck_ || !cv_) throw Error("the cache holds no encoded record");
  ck_->describe(k);
  cv_->describe(v);
}

// Host tables for tests and tools: the rotation signs of (dim, seed), the
// codebook of (dim, bits) and the QJL matrix drawn from key(seed + 1000).
void tq_host_tables(int dim, int bits, int seed, float* signs, float* codebook, float* qjl) {
  if (dim < 2 || dim > 4096) throw Error("dim must be in [2, 4096]");
  if (bits < 1 || bits > 8) throw Error("bits must be in [1, 8]");
  if (signs) {
    const auto s = random_signs(dim, seed);
    std::memcpy(signs, s.data(), s.size() * sizeof(float));
  }
  if (codebook) {
    std::vector<float> cb;
    {
      std::lock_guard<std::mutex> g(g_tq_mutex);
      cb = codebook_host(dim, bits);
    }
    std::memcpy(codebook, cb.data(), cb.size() * sizeof(float));
  }
  if (qjl) {
    const auto S = qjl_matrix(dim, static_cast<uint64_t>(seed) + 1000);
    std::memcpy(qjl, S.data(), S.size() * sizeof(float));
  }
}

}  // namespace vkv

// ------------------------------------------------------------ the C ABI

using namespace vkv;

namespace {
template <class F>
int guarded(F&& f) {
  return guarded_call(std::function<void()>(f));
}
void need_ptr(const void* p, const char* what) {
  if (!p) throw Error(std::string(what) + " must not be NULL");
}
TurboQuantCache* as_tq(vkv_cache c) {
  need_ptr(c, "cache");
  auto* t = dynamic_cast<TurboQuantCache*>(c->impl.get());
  if (!t) throw Error("the cache is not a TurboQuantKVCache");
  return t;
}
vkv_cache wrap(std::unique_ptr<Cache> c) {
  auto* h = new vkv_cache_s;
  h->impl = std::move(c);
  return h;
}
}  // namespace

extern "C" {

int vkv_turboquant_create(int32_t key_bits, int32_t value_bits, int32_t sink_tokens,
                          int32_t residual_tokens, vkv_cache* out) {
  return guarded([&] {
    need_ptr(out, "out");
    *out = wrap(std::make_unique<TurboQuantCache>(key_bits, value_bits, sink_tokens, residual_tokens));
  });
}

int vkv_turboquant_to_compilable(vkv_cache tq, void* stream, vkv_cache* out) {
  return guarded([&] {
    need_ptr(out, "out");
    *out = wrap(CompilableTurboQuantCache::from(*as_tq(tq), S(stream)));
  });
}

int vkv_turboquant_from_simple(vkv_cache simple, int32_t key_bits, int32_t value_bits,
                               int32_t sink_tokens, int32_t residual_tokens, void* stream,
                               vkv_cache* out) {
  return guarded([&] {
    need_ptr(simple, "cache");
    need_ptr(out, "out");
    if (!dynamic_cast<SimpleCache*>(simple->impl.get()))
      throw Error("fromSimpleCache needs a KVCacheSimple");
    *out = wrap(TurboQuantCache::from_simple(*simple->impl, key_bits, value_bits, sink_tokens,
                                             residual_tokens, S(stream)));
  });
}

int vkv_turboquant_has_compressible_middle(int64_t token_count, int32_t sink_tokens,
                                           int32_t residual_tokens, int32_t minimum,
                                           int32_t* out) {
  return guarded([&] {
    need_ptr(out, "out");
    *out = TurboQuantCache::has_compressible_middle(token_count, sink_tokens, residual_tokens,
                                                    minimum) ? 1 : 0;
  });
}

int vkv_turboquant_info(vkv_cache cache, vkv_tq_info* info) {
  return guarded([&] {
    need_ptr(info, "info");
    const TurboQuantCache* t = as_tq(cache);
    *info = vkv_tq_info{};
    info->phase = t->phase_;
    info->has_encoded = t->ck_ && t->cv_ ? 1 : 0;
    info->prefix_tokens = t->prefix_;
    info->window_tokens = t->window_;
    info->key_bits = t->key_bits_;
    info->value_bits = t->value_bits_;
    info->sink_tokens = t->sink_;
    info->residual_tokens = t->residual_;
  });
}

int vkv_turboquant_encoded(vkv_cache cache, vkv_tq_encoded* keys, vkv_tq_encoded* values) {
  return guarded([&] {
    need_ptr(keys, "keys");
    need_ptr(values, "values");
    as_tq(cache)->encoded(keys, values);
  });
}

int vkv_turboquant_window(vkv_cache cache, vkv_array* keys, vkv_array* values, int32_t* present) {
  return guarded([&] {
    need_ptr(present, "present");
    vkv_array k{}, v{};
    *present = as_tq(cache)->window_state(&k, &v) ? 1 : 0;
    if (keys) *keys = k;
    if (values) *values = v;
  });
}

int vkv_turboquant_restore_compressed(vkv_cache cache, const vkv_tq_encoded* keys,
                                      const vkv_tq_encoded* values, int64_t source_offset,
                                      const vkv_array* window_keys, const vkv_array* window_values,
                                      void* stream) {
  return guarded([&] {
    need_ptr(keys, "keys");
    need_ptr(values, "values");
    as_tq(cache)->restore_compressed(*keys, *values, source_offset, window_keys, window_values,
                                     S(stream));
  });
}

int vkv_turboquant_restore_decoded(vkv_cache cache, const vkv_array* keys, const vkv_array* values,
                                   int64_t source_offset, void* stream) {
  return guarded([&] {
    need_ptr(keys, "keys");
    need_ptr(values, "values");
    as_tq(cache)->restore_decoded(*keys, *values, source_offset, S(stream));
  });
}

int vkv_turboquant_write_pool(vkv_cache cache, vkv_pool pool, int32_t layer,
                              const int32_t* slot_mapping, int64_t first_token, int64_t n_tokens,
                              void* stream) {
  return guarded([&] {
    need_ptr(pool, "pool");
    TurboQuantCache* t = as_tq(cache);
    const hipStream_t st = S(stream);
    if (n_tokens < 0 || first_token < 0) throw Error("first_token and n_tokens must be >= 0");
    if (n_tokens == 0) return;
    if (!slot_mapping) throw Error("slot_mapping is required");
    // the keys and values update() returns: [B, H, offset, D] views of the
    // unified buffers (decoded prefix, then the exact window)
    vkv_array s[2];
    if (t->state(st, s) < 2) throw Error("the cache is empty");
    if (first_token + n_tokens > s[0].shape[2])
      throw Error("tokens [first_token, first_token + n_tokens) must lie within the cache's offset");
    Pool& P = *pool->impl;
    const bool keys_only = (P.p.flags & VKV_VIEW_KEYS_ONLY) != 0;
    const int64_t B = s[0].shape[0], H = s[0].shape[1];
    if (H != P.p.n_kv_heads || s[0].shape[3] != P.p.head_dim ||
        (!keys_only && s[1].shape[3] != P.p.v_head_dim))
      throw Error("the cache's heads and head dims must match the pool's");
    const int passes = keys_only ? 1 : 2;
    // rows in another dtype than the pool's are cast first (rounded to
    // nearest even; an f32 pool keeps them exactly)
    const bool cast = s[0].dtype != P.p.dtype || (!keys_only && s[1].dtype != P.p.dtype);
    DevBuf tmp;
    if (cast)
      tmp.alloc(static_cast<size_t>(n_tokens * H * (P.p.head_dim + P.p.v_head_dim)) *
                elem_bytes(P.p.dtype));
    for (int64_t b = 0; b < B; b++) {
      vkv_array rows[2]{};
      int64_t off = 0;
      for (int w = 0; w < passes; w++) {
        const vkv_array& a = s[w];
        const int64_t D = a.shape[3];
        const void* src = static_cast<const uint8_t*>(a.data) +
                          (b * a.strides[0] + first_token * a.strides[2]) * elem_bytes(a.dtype);
        vkv_array& r = rows[w];
        r.dtype = P.p.dtype;
        r.ndim = 3;
        r.shape[0] = n_tokens;
        r.shape[1] = H;
        r.shape[2] = D;
        if (a.dtype == P.p.dtype) {
          r.data = const_cast<void*>(src);
          r.strides[0] = a.strides[2];
          r.strides[1] = a.strides[1];
          r.strides[2] = a.strides[3];
        } else {
          void* dst = tmp.bytes() + off * elem_bytes(P.p.dtype);
          off += n_tokens * H * D;
          const int64_t shape[4] = {1, n_tokens, H, D};
          const int64_t sstr[4] = {0, a.strides[2], a.strides[1], a.strides[3]};
          const int64_t dstr[4] = {0, H * D, D, 1};
          launch_cast4d(src, a.dtype, shape, sstr, dst, P.p.dtype, dstr, st);
          r.data = dst;
          r.strides[0] = H * D;
          r.strides[1] = D;
          r.strides[2] = 1;
        }
      }
      P.append(layer, rows[0], keys_only ? nullptr : &rows[1], slot_mapping + b * n_tokens,
               n_tokens, st);
    }
    // the cast rows live until the appends have read them
    if (cast) VKV_HIP(hipStreamSynchronize(st));
  });
}

int vkv_tq_tables(int32_t dim, int32_t bits, int32_t seed, float* signs, float* codebook,
                  float* qjl) {
  return guarded([&] { tq_host_tables(dim, bits, seed, signs, codebook, qjl); });
}

}  // extern "C"
