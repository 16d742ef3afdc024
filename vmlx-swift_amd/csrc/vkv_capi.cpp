// vkv_capi.cpp -- the extern "C" boundary declared in include/vkv.h.
// Every entry point converts C++ exceptions into a non-zero return and a
// thread-local message, the mlx-c convention
// (Libraries/CmlxDistributedShim/MlxCDistributed.cpp:11-28).
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <string>
#include <vector>

#include "vkv_host.h"

using namespace vkv;

namespace {
thread_local std::string g_error;

template <class F>
int guard(F&& f) {
  try {
    f();
    g_error.clear();
    return 0;
  } catch (const std::exception& e) {
    g_error = e.what();
  } catch (...) {
    g_error = "unknown error";
  }
  return 1;
}

void need(const void* p, const char* what) {
  if (!p) throw Error(std::string(what) + " is NULL");
}

bool is_float(int dt) { return dt == VKV_F32 || dt == VKV_F16 || dt == VKV_BF16; }

bool contiguous(const vkv_array& a) {
  int64_t s = 1;
  for (int i = a.ndim - 1; i >= 0; i--) {
    if (a.shape[i] != 1 && a.strides[i] != s) return false;
    s *= a.shape[i];
  }
  return true;
}

int64_t numel(const vkv_array& a) {
  int64_t n = 1;
  for (int i = 0; i < a.ndim; i++) n *= a.shape[i];
  return n;
}

// Right-aligned broadcast of a mask to [B,H,L,T]: element strides, 0 on
// broadcast dims.
void mask_strides(const vkv_array& m, const int64_t* target, int64_t* out) {
  if (m.ndim < 1 || m.ndim > 4) throw Error("mask must have 1 to 4 dims");
  for (int i = 0; i < 4; i++) out[i] = 0;
  for (int i = 0; i < m.ndim; i++) {
    const int ti = 4 - m.ndim + i;
    if (m.shape[i] == target[ti]) out[ti] = m.strides[i];
    else if (m.shape[i] == 1) out[ti] = 0;
    else throw Error("mask shape does not broadcast to [B, H, L, T]");
  }
}

int32_t choose_parts(int64_t rows_x_heads, int64_t max_len, int32_t* part_tokens) {
  const int64_t target_wgs = 2048;
  int64_t parts = std::max<int64_t>(1, (target_wgs + rows_x_heads - 1) / std::max<int64_t>(1, rows_x_heads));
  parts = std::min<int64_t>(parts, std::max<int64_t>(1, (max_len + 31) / 32));
  int64_t pt = (max_len + parts - 1) / parts;
  pt = std::max<int64_t>(32, (pt + 31) / 32 * 32);
  *part_tokens = static_cast<int32_t>(pt);
  return static_cast<int32_t>(std::max<int64_t>(1, (max_len + pt - 1) / pt));
}

constexpr int kGatherPrefillMinL = 16;
// Bytes of the K/V copy of one key window of a gathered chunk (the whole
// context in one window up to this size).
constexpr int64_t kGatherCopyBytes = int64_t{256} << 20;

// Dispatch options (vkv_set_option): process-wide, read with relaxed loads on
// the hot path.  The environment variables of the same names give their
// initial values, read once.
struct Options {
  std::atomic<int64_t> v[VKV_OPTION_COUNT];
  Options() {
    const char* names[VKV_OPTION_COUNT] = {"VKV_GENERIC_ATTENTION", "VKV_DECODE_WAVES",
                                           "VKV_MLA_SPLITS", "VKV_FDECODE_WAVES",
                                           "VKV_GATHER_TOKENS", "VKV_REFERENCE_SOFTMAX",
                                           "VKV_SEPARATE_TOKEN_WRITE"};
    for (int i = 0; i < VKV_OPTION_COUNT; i++) {
      const char* e = getenv(names[i]);
      int64_t x = 0;
      const bool flag = i == VKV_OPTION_GENERIC_ATTENTION || i == VKV_OPTION_REFERENCE_SOFTMAX ||
                        i == VKV_OPTION_SEPARATE_TOKEN_WRITE;
      if (e) x = flag ? (atoi(e) != 0) : std::max(1, atoi(e));
      v[i].store(x, std::memory_order_relaxed);
    }
  }
};
Options& options() {
  static Options o;
  return o;
}
int64_t option(int which) { return options().v[which].load(std::memory_order_relaxed); }

// Split-K scratch: the per-stream workspace, or (noalloc) the fixed device
// array of the no-allocation entry point.
float* workspace(hipStream_t st, size_t floats, bool noalloc) {
  return noalloc ? decode_scratch(floats) : attention_workspace(st, floats);
}

// Quantized attention with the reference's arithmetic (vkv_refattn.hip):
// the query positions go in batches whose score rows fit 256 MiB.
constexpr int64_t kRefScoreBytes = int64_t{256} << 20;
void run_ref_attention(int dtype, int bits, int group, const AttnArgs& a, int64_t rows,
                       hipStream_t st, bool noalloc) {
  const int64_t B = rows / a.L, T = a.kv.T;
  RefArgs r{};
  r.a = a;
  r.group = group;
  r.bits = bits;
  r.deq_round = a.L >= kGatherPrefillMinL;  // the quantized matmul's tiled path
  r.score_f32 = a.mask_mode == 3 && a.mask_dtype == VKV_F32;  // an f32 additive mask
  r.tpad = (std::max<int64_t>(T, 1) + 63) / 64 * 64;
  const int rep = a.Hq / a.Hkv;
  const int64_t per_l = B * a.Hq * r.tpad;  // score floats per query position
  const int64_t nl = std::max<int64_t>(1, std::min<int64_t>(a.L, kRefScoreBytes / 4 / per_l));
  for (int64_t l0 = 0; l0 < a.L; l0 += nl) {
    r.l0 = static_cast<int32_t>(l0);
    r.nl = static_cast<int32_t>(std::min<int64_t>(nl, a.L - l0));
    r.n_rows = B * a.Hq * r.nl;
    r.part_tokens = ref_part_tokens(B, a.Hkv, rep * r.nl, T, &r.n_parts);
    const size_t sc_floats = static_cast<size_t>(r.n_rows * r.tpad);
    const size_t pv_floats = r.n_parts > 1 ? static_cast<size_t>(r.n_parts * r.n_rows * a.Dv) : 0;
    float* ws = workspace(st, sc_floats + pv_floats, noalloc);
    r.sc = ws;
    r.ws = ws + sc_floats;
    launch_ref_attention(dtype, r, B, st);
  }
}

void run_attention(int dtype, int bits, int group, bool qsem, AttnArgs& a, int64_t rows,
                   int64_t max_len, hipStream_t st, bool noalloc = false) {
  a.group = group;
  if (qsem && bits > 0 && option(VKV_OPTION_REFERENCE_SOFTMAX)) {
    if (a.D > kMaxRefD || a.Dv > kMaxRefD) throw Error("head dims above 256 are not supported here");
    if (rows > 0) run_ref_attention(dtype, bits, group, a, rows, st, noalloc);
    return;
  }
  if (fdecode_supported(dtype, bits, qsem, a) && !option(VKV_OPTION_GENERIC_ATTENTION)) {
    // a small launch: one workgroup per (row, head group), merged in LDS
    // (the fdecode_waves option, a tuning override, keeps the split launch)
    a.wg_parts = option(VKV_OPTION_FDECODE_WAVES)
                     ? 0
                     : fdecode_wg_parts(rows, a.Hq, a.Hkv, max_len, a.D, dtype, &a.part_tokens);
    if (a.wg_parts > 0) {
      a.n_parts = a.wg_parts;
      launch_fdecode(dtype, a, rows, st);
      return;
    }
    a.n_parts = fdecode_parts(rows * a.Hkv, max_len, &a.part_tokens,
                              static_cast<int>(option(VKV_OPTION_FDECODE_WAVES)));
    if (a.n_parts > 1) {
      const size_t per = static_cast<size_t>(rows) * a.Hq * a.n_parts;
      float* ws = workspace(st, per * (a.Dv + 2), noalloc);
      a.ws_o = ws;
      a.ws_ml = ws + per * a.Dv;
      // the merge inside the decode launch where the last part's merge is
      // small (18 parts x 128 dims x 4 heads, one f16 row: step 19.4 -> 17.8
      // us); larger ones keep the separate merge (config 4's window layer,
      // 32 parts x 256 dims x 2 heads: 19.9 us with it, 25.1 inside), as
      // does the no-allocation path, which has no counters
      if (!noalloc && fdecode_merge_here(a.n_parts, a.Dv, a.Hq, a.Hkv))
        a.counters = attention_counters(st, static_cast<size_t>(rows) *
                                                fdecode_counter_count(a.Hq, a.Hkv));
    }
    launch_fdecode(dtype, a, rows, st);
    return;
  }
  // Quantized or paged K/V with a chunk of query tokens (uniform or ragged
  // lengths): gather them to dense rows of the dtype (the dequantized values
  // the reference's dequantize produces; a ragged row fills its own length),
  // then the matrix-core multi-query kernel on the copy.  Fewer query tokens
  // stay on the generic kernel, which keeps the dequantized values
  // unrounded (fp32) as the quantized matmul of the oracle does.
  if ((bits > 0 || a.kv.table) && a.L >= kGatherPrefillMinL && a.kv.T > 0 &&
      !option(VKV_OPTION_GENERIC_ATTENTION)) {
    AttnArgs d = a;
    const int64_t batch = rows / a.L, T = a.kv.T;
    const int64_t es = elem_bytes(dtype);
    const int64_t per_head = T * a.D * es;
    d.kv = KVSrc{};
    d.kv.T = a.kv.T;
    d.kv.seq_lens = a.kv.seq_lens;
    d.kv.kc = Comp{nullptr, a.Hkv * per_head, per_head, a.D * es};
    d.kv.vc = d.kv.kc;
    // a stand-in base with the copy's alignment decides support first
    d.kv.kc.ptr = d.kv.vc.ptr = reinterpret_cast<const uint8_t*>(uintptr_t{256});
    if (a.D == a.Dv && prefill_supported(dtype, 0, d)) {
      d.n_parts = prefill_parts(batch, a.Hkv, a.L, a.Hq / a.Hkv, T, a.D, &d.part_tokens);
      // key windows of whole parts, each gathered to a copy of at most
      // kGatherCopyBytes (or the gather_tokens option) before its parts run
      const int64_t tok_bytes = 2 * batch * a.Hkv * a.D * es;  // K + V per token
      int64_t win = option(VKV_OPTION_GATHER_TOKENS);
      if (win <= 0) win = kGatherCopyBytes / tok_bytes;
      win = std::max<int64_t>(32, win / 32 * 32);
      if (win < T && d.part_tokens > win) {
        d.part_tokens = static_cast<int32_t>(win);
        d.n_parts = static_cast<int32_t>((T + win - 1) / win);
      }
      const int ppw = static_cast<int>(std::max<int64_t>(1, win / d.part_tokens));
      const int64_t wtok = std::min<int64_t>(T, static_cast<int64_t>(ppw) * d.part_tokens);
      const int64_t wbytes = batch * a.Hkv * wtok * a.D * es;  // one matrix of a window
      const size_t copy_floats = static_cast<size_t>((2 * wbytes + 255) / 256 * 64);
      const size_t per = static_cast<size_t>(rows) * a.Hq * d.n_parts;
      float* ws = workspace(st, copy_floats + (d.n_parts > 1 ? per * (a.Dv + 2) : 0), noalloc);
      uint8_t* kd = reinterpret_cast<uint8_t*>(ws);
      uint8_t* vd = kd + wbytes;
      const int64_t wph = wtok * a.D * es;  // copy bytes per (row, kv head)
      d.kv.kc = Comp{kd, a.Hkv * wph, wph, a.D * es};
      d.kv.vc = Comp{vd, a.Hkv * wph, wph, a.D * es};
      if (d.n_parts > 1) {
        d.ws_o = ws + copy_floats;
        d.ws_ml = d.ws_o + per * a.Dv;
      }
      for (int p0 = 0; p0 < d.n_parts; p0 += ppw) {
        GatherArgs g{};
        g.kv = a.kv;
        g.n_seqs = static_cast<int32_t>(batch);
        g.H = a.Hkv;
        g.t_begin = static_cast<int32_t>(static_cast<int64_t>(p0) * d.part_tokens);
        // the copy's layout holds wtok tokens per (row, head); the gather
        // fills each row's tokens of the window (fewer in the last one)
        g.T = static_cast<int32_t>(wtok);
        g.D = a.D;
        g.bits = bits;
        g.group = group;
        g.dtype = dtype;
        g.out = kd;
        g.out_v = vd;
        launch_gather(g, 0, st);
        d.part0 = p0;
        d.parts_run = std::min(ppw, d.n_parts - p0);
        d.t_base = g.t_begin;
        launch_prefill(dtype, qsem, d, batch, st, /*combine=*/false);
      }
      if (d.n_parts > 1) launch_attn_combine(dtype, d, rows, st);
      return;
    }
  }
  if (prefill_supported(dtype, bits, a) && !option(VKV_OPTION_GENERIC_ATTENTION)) {
    const int64_t batch = rows / a.L;
    a.n_parts = prefill_parts(batch, a.Hkv, a.L, a.Hq / a.Hkv, a.kv.T, a.D, &a.part_tokens);
    if (a.n_parts > 1) {
      const size_t per = static_cast<size_t>(rows) * a.Hq * a.n_parts;
      float* ws = workspace(st, per * (a.Dv + 2), noalloc);
      a.ws_o = ws;
      a.ws_ml = ws + per * a.Dv;
    }
    launch_prefill(dtype, qsem, a, batch, st);
    return;
  }
  a.n_parts = choose_parts(rows * a.Hkv, max_len, &a.part_tokens);
  if (a.n_parts > 1) {
    const size_t per = static_cast<size_t>(rows) * a.Hq * a.n_parts;
    float* ws = workspace(st, per * (a.Dv + 2), noalloc);
    a.ws_o = ws;
    a.ws_ml = ws + per * a.Dv;
  }
  launch_attention(dtype, bits, group, qsem, a, rows, st);
}

}  // namespace

namespace vkv {
int guarded_call(const std::function<void()>& f) { return guard(f); }
}  // namespace vkv

extern "C" {

const char* vkv_last_error(void) { return g_error.c_str(); }

int vkv_abi_version(void) { return VKV_ABI_VERSION; }

int vkv_device_count(int32_t* count) {
  return guard([&] {
    need(count, "count");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
  });
}

// ------------------------------------------------------------ quantization

int vkv_quantize_affine(const vkv_array* w, int32_t group_size, int32_t bits, vkv_array* wq,
                        vkv_array* scales, vkv_array* biases, void* stream) {
  return guard([&] {
    need(w, "w");
    need(wq, "wq");
    need(scales, "scales");
    need(biases, "biases");
    if (!is_float(w->dtype)) throw Error("w must be f32, f16 or bf16");
    if (w->ndim < 1 || w->ndim > 4) throw Error("w must have 1 to 4 dims");
    if (w->strides[w->ndim - 1] != 1) throw Error("w last dim must be contiguous");
    const int64_t D = w->shape[w->ndim - 1];
    if (D % group_size) throw Error("last dim must be divisible by group_size");
    const int64_t rows = D ? numel(*w) / D : 0;
    if (wq->dtype != VKV_U32 || numel(*wq) * 32 != rows * D * bits || !contiguous(*wq))
      throw Error("wq must be contiguous u32 with D*bits/32 words per row");
    if (scales->dtype != w->dtype || biases->dtype != w->dtype ||
        numel(*scales) != rows * (D / group_size) || numel(*biases) != numel(*scales) ||
        !contiguous(*scales) || !contiguous(*biases))
      throw Error("scales/biases must be contiguous [..., D/group_size] of w's dtype");
    int64_t e[3] = {1, 1, 1}, s[3] = {0, 0, 0};
    for (int i = 0; i < w->ndim - 1; i++) {
      e[3 - (w->ndim - 1) + i] = w->shape[i];
      s[3 - (w->ndim - 1) + i] = w->strides[i];
    }
    RowSrc src{w->data, e[0], e[1], e[2], s[0], s[1], s[2]};
    RowDst dst{};
    dst.wq = wq->data;
    dst.scales = scales->data;
    dst.biases = biases->data;
    launch_quantize_rows(w->dtype, bits, group_size, 0, src, dst, rows, static_cast<int>(D), S(stream));
  });
}

int vkv_dequantize_affine(const vkv_array* wq, const vkv_array* scales, const vkv_array* biases,
                          int32_t group_size, int32_t bits, vkv_array* out, void* stream) {
  return guard([&] {
    need(wq, "wq");
    need(scales, "scales");
    need(biases, "biases");
    need(out, "out");
    if (!contiguous(*wq) || !contiguous(*scales) || !contiguous(*biases) || !contiguous(*out))
      throw Error("dequantize operands must be contiguous");
    if (bits != 4 && bits != 8) throw Error("bits must be 4 or 8");
    const int64_t D = out->shape[out->ndim - 1];
    const int64_t rows = D ? numel(*out) / D : 0;
    if (numel(*wq) * 32 != rows * D * bits) throw Error("wq does not match out");
    if (out->dtype != scales->dtype || biases->dtype != scales->dtype)
      throw Error("out, scales and biases must share a dtype");
    launch_dequantize(out->dtype, bits, group_size, static_cast<const uint32_t*>(wq->data),
                      scales->data, biases->data, out->data, rows, static_cast<int>(D), S(stream));
  });
}

}  // extern "C"

// ---------------------------------------------------------------- attention

namespace {
// The attention mask arguments: none, causal, or a bool / additive array
// (f32 or the query dtype) broadcast to [B, Hq, L, T].
void set_mask(AttnArgs& a, int32_t mask_mode, const vkv_array* mask, int64_t B, int64_t Hq,
              int64_t L, int64_t T, int q_dtype) {
  if (mask_mode == VKV_MASK_CAUSAL) {
    a.mask_mode = 1;
  } else if (mask_mode == VKV_MASK_ARRAY) {
    need(mask, "mask");
    const int64_t target[4] = {B, Hq, L, T};
    int64_t ms[4];
    mask_strides(*mask, target, ms);
    if (mask->dtype == VKV_BOOL || mask->dtype == VKV_U8) {
      a.mask_mode = 2;
    } else if (mask->dtype == VKV_F32 || mask->dtype == q_dtype) {
      a.mask_mode = 3;
      a.mask_dtype = mask->dtype;
    } else {
      throw Error("mask must be bool, or additive in f32 or the query dtype");
    }
    a.mask = mask->data;
    a.m_sb = ms[0];
    a.m_sh = ms[1];
    a.m_sl = ms[2];
    a.m_st = ms[3];
  } else if (mask_mode != VKV_MASK_NONE) {
    throw Error("unknown mask mode");
  }
}

// Attention sinks: one logit per query head, f32 or the query dtype.
void set_sinks(AttnArgs& a, const vkv_array* sinks, int64_t Hq) {
  if (!sinks) return;
  if (sinks->ndim != 1 || sinks->shape[0] != Hq || (Hq > 1 && sinks->strides[0] != 1))
    throw Error("sinks must be a contiguous [Hq] array");
  if (sinks->dtype != VKV_F32 && sinks->dtype != VKV_F16 && sinks->dtype != VKV_BF16)
    throw Error("sinks must be f32, f16 or bf16");
  if (!sinks->data) throw Error("sinks has no data");
  a.sinks = sinks->data;
  a.sinks_dtype = sinks->dtype;
}
// MLXFast SDPA (vkv_sdpa); pt: a cache update's deferred one-token write,
// which the float decode kernel performs as it reads the token (or, where
// that kernel does not run, a copy launched first).
void sdpa_impl(const vkv_array* q, const vkv_array* k, const vkv_array* v, float scale,
             int32_t mask_mode, const vkv_array* mask, const vkv_array* sinks, vkv_array* out,
             void* stream, Cache* pt) {
  need(q, "q");
  need(k, "k");
  need(v, "v");
  need(out, "out");
  if (q->ndim != 4 || k->ndim != 4 || v->ndim != 4 || out->ndim != 4)
    throw Error("q, k, v and out must be 4-D");
  if (q->dtype != k->dtype || q->dtype != v->dtype || q->dtype != out->dtype || !is_float(q->dtype))
    throw Error("q, k, v and out must share a float dtype");
  if (q->strides[3] != 1 || k->strides[3] != 1 || v->strides[3] != 1 || out->strides[3] != 1)
    throw Error("last dims must be contiguous");
  const int64_t B = q->shape[0], Hq = q->shape[1], L = q->shape[2], D = q->shape[3];
  const int64_t Hkv = k->shape[1], T = k->shape[2], Dv = v->shape[3];
  if (k->shape[0] != B || v->shape[0] != B || v->shape[1] != Hkv || v->shape[2] != T ||
      k->shape[3] != D || Hq % Hkv)
    throw Error("q/k/v shapes are inconsistent");
  if (out->shape[0] != B || out->shape[1] != Hq || out->shape[2] != L || out->shape[3] != Dv)
    throw Error("out must be [B, Hq, L, Dv]");
  const int es = elem_bytes(q->dtype);
  AttnArgs a{};
  a.q = q->data;
  a.q_sb = q->strides[0];
  a.q_sh = q->strides[1];
  a.q_sl = q->strides[2];
  a.L = static_cast<int32_t>(L);
  a.Hq = static_cast<int32_t>(Hq);
  a.Hkv = static_cast<int32_t>(Hkv);
  a.D = static_cast<int32_t>(D);
  a.Dv = static_cast<int32_t>(Dv);
  a.scale = scale;
  a.kv.kc = Comp{static_cast<const uint8_t*>(k->data), k->strides[0] * es, k->strides[1] * es,
                 k->strides[2] * es};
  a.kv.vc = Comp{static_cast<const uint8_t*>(v->data), v->strides[0] * es, v->strides[1] * es,
                 v->strides[2] * es};
  a.kv.T = static_cast<int32_t>(T);
  a.out = out->data;
  a.o_sb = out->strides[0];
  a.o_sh = out->strides[1];
  a.o_sl = out->strides[2];
  set_mask(a, mask_mode, mask, B, Hq, L, T, q->dtype);
  set_sinks(a, sinks, Hq);
  if (pt && pt->pending.set) {
    const Cache::PendingToken& p = pt->pending;
    const vkv_array& nk = p.k;
    const vkv_array& nv = p.v;
    const bool al = reinterpret_cast<uintptr_t>(nk.data) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(nv.data) % 16 == 0 &&
                    (nk.strides[0] * es) % 16 == 0 && (nk.strides[1] * es) % 16 == 0 &&
                    (nv.strides[0] * es) % 16 == 0 && (nv.strides[1] * es) % 16 == 0;
    const bool same = k->data == p.dk->buf->get() && v->data == p.dv->buf->get() &&
                      nk.dtype == q->dtype && nv.dtype == q->dtype;
    if (al && same && p.pos < T && fdecode_supported(q->dtype, 0, false, a) &&
        !option(VKV_OPTION_GENERIC_ATTENTION)) {
      a.has_new = 1;
      a.new_t = p.pos;
      a.nk_ptr = static_cast<const uint8_t*>(nk.data);
      a.nv_ptr = static_cast<const uint8_t*>(nv.data);
      a.nk_sb = nk.strides[0] * es;
      a.nk_sh = nk.strides[1] * es;
      a.nv_sb = nv.strides[0] * es;
      a.nv_sh = nv.strides[1] * es;
      pt->pending.set = false;  // the decode kernel writes it
    } else {
      pt->flush_pending(S(stream));
    }
  }
  run_attention(q->dtype, 0, 64, false, a, B * L, T, S(stream));
}

}  // namespace

extern "C" {

int vkv_sdpa(const vkv_array* q, const vkv_array* k, const vkv_array* v, float scale,
             int32_t mask_mode, const vkv_array* mask, const vkv_array* sinks, vkv_array* out,
             void* stream) {
  return guard([&] { sdpa_impl(q, k, v, scale, mask_mode, mask, sinks, out, stream, nullptr); });
}
int vkv_quantized_sdpa(const vkv_array* q, const vkv_array* k_wq, const vkv_array* k_scales,
                       const vkv_array* k_biases, const vkv_array* v_wq, const vkv_array* v_scales,
                       const vkv_array* v_biases, int32_t group_size, int32_t bits, float scale,
                       int32_t mask_mode, const vkv_array* mask, vkv_array* out, void* stream) {
  return guard([&] {
    const vkv_array* arrs[6] = {k_wq, k_scales, k_biases, v_wq, v_scales, v_biases};
    need(q, "q");
    need(out, "out");
    for (auto* x : arrs) {
      need(x, "quantized tuple array");
      if (x->ndim != 4 || x->strides[3] != 1) throw Error("quantized tuples must be 4-D, last dim contiguous");
    }
    if (group_size != 32 && group_size != 64 && group_size != 128)
      throw Error("quantized attention supports group_size 32, 64 or 128");
    if (bits != 4 && bits != 8) throw Error("bits must be 4 or 8");
    if (q->ndim != 4 || out->ndim != 4 || q->strides[3] != 1 || out->strides[3] != 1)
      throw Error("q and out must be 4-D with a contiguous last dim");
    if (!is_float(q->dtype)) throw Error("q must be f32, f16 or bf16");
    const int64_t B = q->shape[0], Hq = q->shape[1], L = q->shape[2], D = q->shape[3];
    const int64_t Hkv = k_wq->shape[1], T = k_wq->shape[2];
    if (D % group_size || (D * bits) % 32) throw Error("head dim must be a multiple of group_size");
    if (Hkv < 1 || Hq % Hkv) throw Error("query heads must be a multiple of kv heads");
    // all six tuple arrays are [B, Hkv, T, last]: codes last = D*bits/32
    // (u32), scales and biases last = D/group_size (q's dtype)
    for (int i = 0; i < 6; i++) {
      const vkv_array* x = arrs[i];
      const bool codes = i % 3 == 0;
      if (x->shape[0] != B || x->shape[1] != Hkv || x->shape[2] != T ||
          x->shape[3] != (codes ? D * bits / 32 : D / group_size))
        throw Error(std::string("quantized tuple ") + (i < 3 ? "keys" : "values") +
                    (codes ? " wq" : i % 3 == 1 ? " scales" : " biases") +
                    " must be [B, Hkv, T, " + (codes ? "D*bits/32]" : "D/group_size]") +
                    " matching q and the keys");
      if (codes ? x->dtype != VKV_U32 : x->dtype != q->dtype)
        throw Error(codes ? "quantized codes must be u32"
                          : "q, scales and biases must share a dtype");
      if (!x->data && B * Hkv * T > 0) throw Error("quantized tuple array has no data");
    }
    if (out->dtype != q->dtype) throw Error("out must have q's dtype");
    if (out->shape[0] != B || out->shape[1] != Hq || out->shape[2] != L || out->shape[3] != D)
      throw Error("out must be [B, Hq, L, D]");
    const int es = elem_bytes(q->dtype);
    AttnArgs a{};
    a.q = q->data;
    a.q_sb = q->strides[0];
    a.q_sh = q->strides[1];
    a.q_sl = q->strides[2];
    a.L = static_cast<int32_t>(L);
    a.Hq = static_cast<int32_t>(Hq);
    a.Hkv = static_cast<int32_t>(Hkv);
    a.D = static_cast<int32_t>(D);
    a.Dv = static_cast<int32_t>(D);
    a.scale = scale;
    auto comp = [&](const vkv_array* x, int esz) {
      return Comp{static_cast<const uint8_t*>(x->data), x->strides[0] * esz, x->strides[1] * esz,
                  x->strides[2] * esz};
    };
    a.kv.kc = comp(k_wq, 4);
    a.kv.ks = comp(k_scales, es);
    a.kv.kb = comp(k_biases, es);
    a.kv.vc = comp(v_wq, 4);
    a.kv.vs = comp(v_scales, es);
    a.kv.vb = comp(v_biases, es);
    a.kv.T = static_cast<int32_t>(T);
    a.out = out->data;
    a.o_sb = out->strides[0];
    a.o_sh = out->strides[1];
    a.o_sl = out->strides[2];
    set_mask(a, mask_mode, mask, B, Hq, L, T, q->dtype);
    run_attention(q->dtype, bits, group_size, true, a, B * L, T, S(stream));
  });
}

}  // extern "C"

namespace {
// The router's decode token over a QuantizedKVCache: its key / value rows
// [B, Hkv, D] (element strides), which the matrix-core decode launch
// quantizes and writes into the pool itself.
struct DecodeToken {
  const void* k;
  const void* v;
  int64_t k_ss, k_sh, v_ss, v_sh;
};

// Whether a paged decode call (3-D q / out checked by the caller) runs on
// the matrix-core kernel (vkv_decode.hip).
bool paged_decode_on_matrix_cores(const vkv_array* q, const vkv_array* out,
                                  const vkv_paged_view* kv) {
  const bool keys_only = (kv->flags & VKV_VIEW_KEYS_ONLY) != 0;
  const int rep = static_cast<int>(q->shape[1] / kv->n_kv_heads);
  // the matrix-core kernel loads queries 16 bytes and stores outputs 8
  // bytes at a time
  const bool aligned = (reinterpret_cast<uintptr_t>(q->data) % 16 == 0) &&
                       q->strides[0] % 8 == 0 && q->strides[1] % 8 == 0 &&
                       (reinterpret_cast<uintptr_t>(out->data) % 8 == 0) &&
                       out->strides[0] % 4 == 0 && out->strides[1] % 4 == 0;
  // (the matrix-core reference path stores bf16 score rows of group-64
  // caches: an f16 or group-128 cache with the reference softmax takes the
  // generic reference path)
  return kv->bits > 0 && !keys_only && aligned && kv->max_len <= qdecode_max_len() &&
         !option(VKV_OPTION_GENERIC_ATTENTION) &&
         !(option(VKV_OPTION_REFERENCE_SOFTMAX) && (kv->dtype != VKV_BF16 || kv->group_size != 64)) &&
         qdecode_supported(kv->dtype, kv->bits, kv->head_dim, kv->block_size, rep, kv->group_size);
}

// vkv_paged_sdpa and its no-allocation variant (noalloc: split-K partials in
// the fixed scratch array, nothing allocated); tok: the router's decode
// token, which the matrix-core launch writes.
void paged_sdpa(const vkv_array* q, const vkv_paged_view* kv, float scale, vkv_array* out,
                void* stream, bool noalloc, const DecodeToken* tok = nullptr) {
  {
    need(q, "q");
    need(kv, "kv");
    need(out, "out");
    if (q->ndim != 3 || out->ndim != 3 || q->strides[2] != 1 || out->strides[2] != 1)
      throw Error("q and out must be [n_seqs, Hq, D] with a contiguous last dim");
    if (q->dtype != kv->dtype || out->dtype != kv->dtype) throw Error("q/out dtype must match the view");
    if (q->shape[0] != kv->n_seqs || q->shape[2] != kv->head_dim || out->shape[0] != kv->n_seqs ||
        out->shape[1] != q->shape[1] || out->shape[2] != kv->v_head_dim)
      throw Error("q/out shapes do not match the view");
    if (q->shape[1] % kv->n_kv_heads) throw Error("query heads must be a multiple of kv heads");
    if (!kv->block_table) throw Error("view has no block table");
    const int rep = static_cast<int>(q->shape[1] / kv->n_kv_heads);
    if (paged_decode_on_matrix_cores(q, out, kv)) {
      // matrix-core path (vkv_decode.hip)
      KVSrc src = kvsrc_from_view(*kv);
      DecodeArgs d{};
      d.q = static_cast<const uint16_t*>(q->data);
      d.q_ss = q->strides[0];
      d.q_sh = q->strides[1];
      d.out = static_cast<uint16_t*>(out->data);
      d.o_ss = out->strides[0];
      d.o_sh = out->strides[1];
      d.scale = scale;
      d.base = src.base;
      d.block_bytes = src.block_bytes;
      d.head_bytes = src.head_bytes;
      d.kc_off = src.kc_off;
      d.vc_off = src.vc_off;
      d.sb_off = src.sb_off;
      d.table = kv->block_table;
      d.table_stride = kv->table_stride;
      d.block_size = kv->block_size;
      d.seq_lens = kv->seq_lens;
      d.max_len = kv->max_len;
      d.Hq = static_cast<int32_t>(q->shape[1]);
      d.Hkv = kv->n_kv_heads;
      d.rep = rep;
      d.n_seqs = kv->n_seqs;
      const int want = static_cast<int>(option(VKV_OPTION_DECODE_WAVES));
      d.n_waves = want;  // 0 = choose per launch
      const int chunk = std::min(kv->n_seqs, qdecode_max_seqs());
      const size_t part_floats =
          qdecode_workspace_floats(chunk, kv->n_kv_heads, rep, kv->head_dim, kv->max_len);
      const bool ref = option(VKV_OPTION_REFERENCE_SOFTMAX) != 0;
      d.dtype = kv->dtype;
      d.group = kv->group_size;
      // the reference path's bf16 score rows follow the partials
      d.sc_stride = (std::max<int64_t>(kv->max_len, 1) + 63) / 64 * 64;
      const size_t sc_floats = ref ? static_cast<size_t>(chunk) * d.Hq * d.sc_stride / 2 : 0;
      d.ws = workspace(S(stream), (part_floats + 63) / 64 * 64 + sc_floats, noalloc);
      d.sc = ref ? reinterpret_cast<uint16_t*>(d.ws + (part_floats + 63) / 64 * 64) : nullptr;
      // counters of the merge inside the launch, where the launch takes it
      // (the no-allocation entry point has none: its partials merge in the
      // separate launch, with the same arithmetic)
      if (!noalloc && !ref && kv->head_dim <= 128)
        d.counters = attention_counters(S(stream), static_cast<size_t>(chunk) * kv->n_kv_heads *
                                                       qdecode_head_groups(rep));
      if (tok) {
        if (ref) throw Error("the decode token needs the fused decode");
        d.new_k = static_cast<const uint16_t*>(tok->k);
        d.new_v = static_cast<const uint16_t*>(tok->v);
        d.nk_ss = tok->k_ss;
        d.nk_sh = tok->k_sh;
        d.nv_ss = tok->v_ss;
        d.nv_sh = tok->v_sh;
      }
      launch_qdecode(d, kv->bits, kv->head_dim, S(stream), ref);
      return;
    }
    if (tok) throw Error("the decode token needs the matrix-core decode");
    AttnArgs a{};
    a.q = q->data;
    a.q_sb = q->strides[0];
    a.q_sh = q->strides[1];
    a.q_sl = 0;
    a.L = 1;
    a.Hq = static_cast<int32_t>(q->shape[1]);
    a.Hkv = kv->n_kv_heads;
    a.D = kv->head_dim;
    a.Dv = kv->v_head_dim;
    a.scale = scale;
    a.kv = kvsrc_from_view(*kv);
    a.out = out->data;
    a.o_sb = out->strides[0];
    a.o_sh = out->strides[1];
    a.o_sl = 0;
    run_attention(kv->dtype, kv->bits, kv->group_size, kv->bits > 0, a, kv->n_seqs, kv->max_len,
                  S(stream), noalloc);
  }
}
}  // namespace

extern "C" {

int vkv_paged_sdpa(const vkv_array* q, const vkv_paged_view* kv, float scale, vkv_array* out,
                   void* stream) {
  return guard([&] { paged_sdpa(q, kv, scale, out, stream, false); });
}

int vkv_paged_sdpa_noalloc(const vkv_array* q, const vkv_paged_view* kv, float scale,
                           vkv_array* out, void* stream) {
  return guard([&] { paged_sdpa(q, kv, scale, out, stream, true); });
}

int vkv_workspace_release(void* stream, int64_t* bytes) {
  return guard([&] {
    const size_t n = workspace_release(S(stream));
    if (bytes) *bytes = static_cast<int64_t>(n);
  });
}

int vkv_quantized_paged_sdpa(const vkv_array* q, const vkv_paged_view* kv, float scale,
                             int32_t mask_mode, const vkv_array* mask, vkv_array* out,
                             void* stream) {
  return guard([&] {
    need(q, "q");
    need(kv, "kv");
    need(out, "out");
    auto call = [](int rc) {
      if (rc != 0) throw Error(g_error);
    };
    const vkv_paged_view& view = *kv;
    if (view.bits != 4 && view.bits != 8) throw Error("the view must hold affine 4- or 8-bit blocks");
    if (view.flags & VKV_VIEW_KEYS_ONLY) throw Error("a keys-only view has no values");
    if (q->ndim != 4 || out->ndim != 4) throw Error("q and out must be 4-D");
    const int64_t B = q->shape[0], Hq = q->shape[1], L = q->shape[2];
    if (q->dtype != view.dtype || out->dtype != view.dtype) throw Error("q/out dtype must match the view");
    if (q->shape[3] != view.head_dim || out->shape[0] != B || out->shape[1] != Hq ||
        out->shape[2] != L || out->shape[3] != view.v_head_dim || B != view.n_seqs ||
        view.n_kv_heads < 1 || Hq % view.n_kv_heads)
      throw Error("q/out shapes do not match the view");
    if (L == 1 && mask_mode == VKV_MASK_NONE) {
      // one decode token: the paged decode path over [B, Hq, D] views
      vkv_array q3 = *q, o3 = *out;
      q3.ndim = o3.ndim = 3;
      q3.shape[2] = q->shape[3];
      q3.strides[2] = q->strides[3];
      o3.shape[2] = out->shape[3];
      o3.strides[2] = out->strides[3];
      call(vkv_paged_sdpa(&q3, &view, scale, &o3, stream));
      return;
    }
    if (q->strides[3] != 1 || out->strides[3] != 1) throw Error("last dims must be contiguous");
    AttnArgs a{};
    a.q = q->data;
    a.q_sb = q->strides[0];
    a.q_sh = q->strides[1];
    a.q_sl = q->strides[2];
    a.L = static_cast<int32_t>(L);
    a.Hq = static_cast<int32_t>(Hq);
    a.Hkv = view.n_kv_heads;
    a.D = view.head_dim;
    a.Dv = view.v_head_dim;
    a.scale = scale;
    a.kv = kvsrc_from_view(view);
    a.out = out->data;
    a.o_sb = out->strides[0];
    a.o_sh = out->strides[1];
    a.o_sl = out->strides[2];
    set_mask(a, mask_mode, mask, B, Hq, L, view.max_len, view.dtype);
    run_attention(view.dtype, view.bits, view.group_size, true, a, B * L, view.max_len, S(stream));
  });
}

}  // extern "C"

namespace {

// The router's one-token decode step over a QuantizedKVCache in one launch:
// updateQuantized's bookkeeping on the host, then the matrix-core decode,
// which quantizes the token and stores it into its block before reading it
// (the same bits as the append launch it replaces).  Returns false, having
// done nothing, where that launch would not run (other shapes, options or
// alignments take the two-call path).
bool quantized_decode_step(const vkv_array* q, const vkv_array* keys, const vkv_array* values,
                           vkv_cache cache, float scale, int32_t mask_mode, vkv_array* out,
                           void* stream) {
  auto* qc = dynamic_cast<QuantizedCache*>(cache->impl.get());
  if (!qc || option(VKV_OPTION_SEPARATE_TOKEN_WRITE) || mask_mode != VKV_MASK_NONE) return false;
  if (q->ndim != 4 || out->ndim != 4 || q->shape[2] != 1 || keys->ndim != 4 || values->ndim != 4 ||
      keys->shape[2] != 1 || values->shape[2] != 1 || keys->dtype != values->dtype ||
      q->strides[3] != 1 || out->strides[3] != 1)
    return false;
  // an existing store of the token's geometry (a first update takes the
  // two-call path, which creates it), 4- or 8-bit g64, and one head group
  // per kv head (at most 8 query heads a kv head): with two, two waves
  // would write the token's 4-bit value nibbles, whose clear-then-set
  // atomics one could read between
  if (q->shape[1] > 8 * keys->shape[1]) return false;
  if (!qc->store_.get() || keys->dtype != qc->dtype_ || keys->shape[0] != qc->B_ ||
      keys->shape[1] != qc->H_ || keys->shape[3] != qc->D_ || values->shape[0] != qc->B_ ||
      values->shape[1] != qc->H_ || values->shape[3] != qc->D_ || qc->group_ != 64 ||
      (qc->bits_ != 4 && qc->bits_ != 8) || option(VKV_OPTION_REFERENCE_SOFTMAX))
    return false;
  // 16-byte rows of 8 elements
  for (const vkv_array* a : {keys, values})
    if (reinterpret_cast<uintptr_t>(a->data) % 16 || a->strides[0] % 8 || a->strides[1] % 8 ||
        a->strides[3] != 1)
      return false;
  // the view the step will attend: the current one, one token longer
  vkv_paged_view next = qc->view();
  next.max_len += 1;
  vkv_array q3 = *q, o3 = *out;
  q3.ndim = o3.ndim = 3;
  q3.shape[2] = q->shape[3];
  q3.strides[2] = q->strides[3];
  o3.shape[2] = out->shape[3];
  o3.strides[2] = out->strides[3];
  if (q->dtype != next.dtype || out->dtype != next.dtype || q->shape[0] != next.n_seqs ||
      q->shape[3] != next.head_dim || out->shape[0] != next.n_seqs || out->shape[1] != q->shape[1] ||
      out->shape[3] != next.v_head_dim || q->shape[1] % next.n_kv_heads ||
      !paged_decode_on_matrix_cores(&q3, &o3, &next))
    return false;
  const int64_t prev = qc->advance(*keys, *values, S(stream));
  const vkv_paged_view view = qc->view();
  const DecodeToken tok{keys->data,        values->data,      keys->strides[0],
                        keys->strides[1], values->strides[0], values->strides[1]};
  try {
    paged_sdpa(&q3, &view, scale, &o3, stream, false, &tok);
  } catch (...) {
    // the update stands even where the attention failed (the two-call path
    // writes the token first): the append launch stores it (the same bits
    // the decode launch writes, should that have run)
    qc->write_tokens(*keys, *values, prev, S(stream));
    throw;
  }
  return true;
}

}  // namespace

extern "C" {

int vkv_attention_with_cache_update(const vkv_array* q, const vkv_array* keys, const vkv_array* values,
                                    vkv_cache cache, float scale, int32_t mask_mode,
                                    const vkv_array* mask, const vkv_array* sinks, vkv_array* out,
                                    void* stream) {
  return guard([&] {
    need(q, "q");
    need(keys, "keys");
    need(values, "values");
    need(out, "out");
    auto call = [](int rc) {
      if (rc != 0) throw Error(g_error);
    };
    if (!cache) {  // AttentionUtils.swift:85-93
      call(vkv_sdpa(q, keys, values, scale, mask_mode, mask, sinks, out, stream));
      return;
    }
    if (q->ndim != 4 || out->ndim != 4) throw Error("q and out must be 4-D");
    if (cache->impl->kind() == VKV_CACHE_QUANTIZED) {  // :94-105
      // the quantized path has no sinks (the models refuse them,
      // Libraries/MLXLLM/Models/GPTOSS.swift:223-235)
      if (sinks) throw Error("quantized attention does not support sinks");
      if (quantized_decode_step(q, keys, values, cache, scale, mask_mode, out, stream)) return;
      vkv_paged_view view{};
      call(vkv_cache_update_quantized(cache, keys, values, stream, &view));
      call(vkv_quantized_paged_sdpa(q, &view, scale, mask_mode, mask, out, stream));
      return;
    }
    // :106-142: update, then the cache's array mask when none was given.
    // A one-token update of a KVCacheSimple or RotatingKVCache leaves its
    // copy to the float decode kernel that follows (it writes the token as
    // it reads it); any other path flushes the copy first.
    vkv_array ck{}, cv{};
    Cache* c = cache->impl.get();
    c->defer_token = true;
    const int rc = vkv_cache_update(cache, keys, values, stream, &ck, &cv);
    c->defer_token = false;
    if (rc != 0) {
      c->flush_pending(S(stream));
      throw Error(g_error);
    }
    try {
      int32_t mode = mask_mode;
      const vkv_array* m = mask;
      vkv_array cm{};
      if (mask_mode == VKV_MASK_NONE) {
        const int cmode = c->make_mask(static_cast<int>(q->shape[2]), 0, true, S(stream), &cm);
        if (cmode == VKV_MASK_ARRAY) {
          mode = VKV_MASK_ARRAY;
          m = &cm;
        }
      }
      sdpa_impl(q, &ck, &cv, scale, mode, m, sinks, out, stream, c);
    } catch (...) {
      c->flush_pending(S(stream));
      throw;
    }
    c->flush_pending(S(stream));  // (nothing left once the kernel took it)
  });
}

int vkv_mla_decode(const vkv_array* q, const vkv_paged_view* kv, float scale, vkv_array* out,
                   void* stream) {
  return guard([&] {
    need(q, "q");
    need(kv, "kv");
    need(out, "out");
    if (!(kv->flags & VKV_VIEW_KEYS_ONLY)) throw Error("vkv_mla_decode needs a keys-only (latent) view");
    if (kv->n_kv_heads != 1) throw Error("an MLA latent view has one kv head");
    if (q->ndim != 3 || out->ndim != 3 || q->strides[2] != 1 || out->strides[2] != 1)
      throw Error("q and out must be [n_seqs, H, D] with a contiguous last dim");
    if (q->dtype != kv->dtype || out->dtype != kv->dtype) throw Error("q/out dtype must match the view");
    if (q->shape[0] != kv->n_seqs || q->shape[2] != kv->head_dim || out->shape[0] != kv->n_seqs ||
        out->shape[1] != q->shape[1] || out->shape[2] != kv->v_head_dim)
      throw Error("q/out shapes do not match the view");
    if (!kv->block_table) throw Error("view has no block table");
    const bool aligned = (reinterpret_cast<uintptr_t>(q->data) % 16 == 0) &&
                         q->strides[0] % 8 == 0 && q->strides[1] % 8 == 0;
    // (the matrix-core kernel takes the max of the raw scores, so scale > 0)
    if (!aligned || !(scale > 0.0f) || option(VKV_OPTION_GENERIC_ATTENTION) ||
        !mla_supported(kv->dtype, kv->bits, kv->group_size, kv->head_dim, kv->v_head_dim,
                       kv->n_kv_heads, kv->block_size)) {
      // other latent geometries run on the generic paged kernel
      if (vkv_paged_sdpa(q, kv, scale, out, stream) != 0) throw Error(vkv_last_error());
      return;
    }
    KVSrc src = kvsrc_from_view(*kv);
    if (!mla_layout_supported(src.base, src.block_bytes, src.sb_off)) {
      if (vkv_paged_sdpa(q, kv, scale, out, stream) != 0) throw Error(vkv_last_error());
      return;
    }
    // matrix-core path (vkv_mla.hip)
    MlaArgs m{};
    m.q = static_cast<const uint16_t*>(q->data);
    m.q_ss = q->strides[0];
    m.q_sh = q->strides[1];
    m.out = static_cast<uint16_t*>(out->data);
    m.o_ss = out->strides[0];
    m.o_sh = out->strides[1];
    m.scale = scale;
    m.base = src.base;
    m.block_bytes = src.block_bytes;
    m.sb_off = src.sb_off;
    m.table = kv->block_table;
    m.table_stride = kv->table_stride;
    m.block_size = kv->block_size;
    m.seq_lens = kv->seq_lens;
    m.max_len = kv->max_len;
    m.H = static_cast<int32_t>(q->shape[1]);
    m.n_seqs = kv->n_seqs;
    if (m.H < 1 || m.n_seqs < 1) return;
    const int want = static_cast<int>(option(VKV_OPTION_MLA_SPLITS));
    const size_t ws = mla_plan(m, want);
    if (ws) m.ws_o = reinterpret_cast<uint16_t*>(attention_workspace(S(stream), ws));
    launch_mla(m, S(stream));
  });
}

// ------------------------------------------------------------------ caches

int vkv_cache_create(const vkv_cache_params* params, vkv_cache* out) {
  return guard([&] {
    need(params, "params");
    need(out, "out");
    auto h = new vkv_cache_s;
    h->impl = make_cache(*params);
    *out = h;
  });
}

int vkv_cache_destroy(vkv_cache cache) {
  return guard([&] { delete cache; });
}

int vkv_cache_copy(vkv_cache cache, void* stream, vkv_cache* out) {
  return guard([&] {
    need(cache, "cache");
    need(out, "out");
    auto h = new vkv_cache_s;
    h->impl = cache->impl->copy(S(stream));
    *out = h;
  });
}

int vkv_cache_update(vkv_cache cache, const vkv_array* keys, const vkv_array* values, void* stream,
                     vkv_array* out_keys, vkv_array* out_values) {
  return guard([&] {
    need(cache, "cache");
    if (cache->impl->kind() == VKV_CACHE_QUANTIZED)
      throw Error("`update` was called on `QuantizedKVCache`. Use `updateQuantized` instead.");
    need(keys, "keys");
    need(values, "values");
    need(out_keys, "out_keys");
    need(out_values, "out_values");
    cache->impl->update(*keys, *values, S(stream), out_keys, out_values);
  });
}

int vkv_cache_update_quantized(vkv_cache cache, const vkv_array* keys, const vkv_array* values,
                               void* stream, vkv_paged_view* out) {
  return guard([&] {
    need(cache, "cache");
    need(keys, "keys");
    need(values, "values");
    need(out, "out");
    cache->impl->update_quantized(*keys, *values, S(stream), out);
  });
}

int vkv_cache_update_quantized_tuples(vkv_cache cache, const vkv_array* keys,
                                      const vkv_array* values, void* stream, vkv_array* out) {
  return guard([&] {
    need(cache, "cache");
    need(keys, "keys");
    need(values, "values");
    need(out, "out");
    auto* q = dynamic_cast<QuantizedCache*>(cache->impl.get());
    if (!q) throw Error("updateQuantized needs a QuantizedKVCache");
    vkv_paged_view view{};
    q->update_quantized(*keys, *values, S(stream), &view);
    q->tuples(S(stream), out);
  });
}

int vkv_cache_kind(vkv_cache cache, int32_t* kind) {
  return guard([&] {
    need(cache, "cache");
    need(kind, "kind");
    *kind = cache->impl->kind();
  });
}

int vkv_cache_offset(vkv_cache cache, int64_t* offset) {
  return guard([&] {
    need(cache, "cache");
    need(offset, "offset");
    *offset = cache->impl->current_offset();
  });
}

int vkv_cache_set_offset(vkv_cache cache, int64_t offset) {
  return guard([&] {
    need(cache, "cache");
    cache->impl->set_offset(offset);
  });
}

int vkv_cache_max_size(vkv_cache cache, int64_t* max_size) {
  return guard([&] {
    need(cache, "cache");
    need(max_size, "max_size");
    *max_size = cache->impl->max_size();
  });
}

int vkv_cache_is_trimmable(vkv_cache cache, int32_t* trimmable) {
  return guard([&] {
    need(cache, "cache");
    need(trimmable, "trimmable");
    *trimmable = cache->impl->trimmable() ? 1 : 0;
  });
}

int vkv_cache_trim(vkv_cache cache, int64_t n, int64_t* trimmed) {
  return guard([&] {
    need(cache, "cache");
    int64_t t = cache->impl->trim(n);
    if (trimmed) *trimmed = t;
  });
}

int vkv_cache_capacity(vkv_cache cache, int64_t* capacity) {
  return guard([&] {
    need(cache, "cache");
    need(capacity, "capacity");
    *capacity = cache->impl->capacity();
  });
}

int vkv_cache_state(vkv_cache cache, void* stream, vkv_array* arrays, int32_t* count) {
  return guard([&] {
    need(cache, "cache");
    need(arrays, "arrays");
    need(count, "count");
    *count = cache->impl->state(S(stream), arrays);
  });
}

int vkv_cache_set_state(vkv_cache cache, const vkv_array* arrays, int32_t count, void* stream) {
  return guard([&] {
    need(cache, "cache");
    if (count > 0) need(arrays, "arrays");
    cache->impl->set_state(arrays, count, S(stream));
  });
}

int vkv_cache_meta_state(vkv_cache cache, char* buf, int64_t buf_len, int32_t* count) {
  return guard([&] {
    need(cache, "cache");
    need(buf, "buf");
    need(count, "count");
    auto v = cache->impl->meta_state();
    int64_t need_len = 0;
    for (auto& s : v) need_len += static_cast<int64_t>(s.size()) + 1;
    if (need_len > buf_len) throw Error("metaState buffer too small");
    char* p = buf;
    for (auto& s : v) {
      memcpy(p, s.c_str(), s.size() + 1);
      p += s.size() + 1;
    }
    *count = static_cast<int32_t>(v.size());
  });
}

int vkv_cache_set_meta_state(vkv_cache cache, const char* const* strings, int32_t count) {
  return guard([&] {
    need(cache, "cache");
    std::vector<std::string> v;
    for (int i = 0; i < count; i++) {
      need(strings[i], "metaState string");
      v.emplace_back(strings[i]);
    }
    cache->impl->set_meta_state(v);
  });
}

int vkv_cache_make_mask(vkv_cache cache, int32_t n, int32_t window, int32_t return_array, void* stream,
                        int32_t* mode, vkv_array* mask) {
  return guard([&] {
    need(cache, "cache");
    need(mode, "mode");
    vkv_array m{};
    *mode = cache->impl->make_mask(n, window, return_array != 0, S(stream), &m);
    if (mask) *mask = m;
  });
}

int vkv_set_option(int32_t which, int64_t value) {
  return guard([&] {
    if (which < 0 || which >= VKV_OPTION_COUNT) throw Error("unknown option");
    if (value < 0) throw Error("option values must be >= 0");
    options().v[which].store(value, std::memory_order_relaxed);
  });
}

int vkv_get_option(int32_t which, int64_t* value) {
  return guard([&] {
    if (which < 0 || which >= VKV_OPTION_COUNT) throw Error("unknown option");
    need(value, "value");
    *value = option(which);
  });
}

int vkv_batch_causal_mask(int32_t n, const int32_t* offsets, const int32_t* key_lens, int32_t batch,
                          int32_t window, void* out, int64_t out_bytes, void* stream,
                          int32_t* max_total) {
  return guard([&] {
    if (batch <= 0) throw Error("createBatchCausalMask requires at least one sequence");
    if (n < 0) throw Error("queryLen must be >= 0");
    need(offsets, "offsets");
    need(max_total, "max_total");
    std::vector<int32_t> kl(batch);
    int64_t mx = 0;
    for (int b = 0; b < batch; ++b) {
      if (offsets[b] < 0) throw Error("offsets must be >= 0");
      const int64_t len = key_lens ? key_lens[b] : static_cast<int64_t>(offsets[b]) + n;
      if (len < 0 || len > INT32_MAX) throw Error("key lengths must be in [0, 2^31)");
      kl[b] = static_cast<int32_t>(len);
      mx = std::max(mx, len);
    }
    *max_total = static_cast<int32_t>(mx);
    if (!out) return;
    const int64_t bytes = static_cast<int64_t>(batch) * n * mx;
    if (out_bytes < bytes) throw Error("the mask buffer holds fewer than batch * n * max_total bytes");
    launch_batch_mask(n, static_cast<int>(mx), window, offsets, kl.data(), batch,
                      static_cast<uint8_t*>(out), S(stream));
  });
}

int vkv_cache_to_quantized(vkv_cache simple, int32_t group_size, int32_t bits, void* stream,
                           vkv_cache* out) {
  return guard([&] {
    need(simple, "cache");
    need(out, "out");
    auto* s = dynamic_cast<SimpleCache*>(simple->impl.get());
    if (!s) throw Error("toQuantized needs a KVCacheSimple");
    auto h = new vkv_cache_s;
    try {
      h->impl = s->to_quantized(group_size > 0 ? group_size : 64, bits > 0 ? bits : 4, S(stream));
    } catch (...) {
      delete h;
      throw;
    }
    *out = h;
  });
}

int vkv_cache_to_compilable(vkv_cache src, int64_t max_length, void* stream, vkv_cache* out) {
  return guard([&] {
    need(src, "cache");
    need(out, "out");
    if (max_length <= 0) throw Error("maxLength must be > 0");
    auto c = std::make_unique<CompilableCache>(max_length, 256);
    vkv_array s[6];
    const int n = src->impl->state(S(stream), s);
    c->init_from(s, n, S(stream));
    auto h = new vkv_cache_s;
    h->impl = std::move(c);
    *out = h;
  });
}

int vkv_cache_to_compilable_rotating(vkv_cache rotating, void* stream, vkv_cache* out) {
  return guard([&] {
    need(rotating, "cache");
    need(out, "out");
    if (rotating->impl->kind() != VKV_CACHE_ROTATING)
      throw Error("CompilableRotatingKVCache(from:) needs a RotatingKVCache");
    const auto* r = static_cast<const RotatingCache*>(rotating->impl.get());
    auto c = std::make_unique<CompilableRotatingCache>(static_cast<int>(r->max_), static_cast<int>(r->keep_),
                                                       static_cast<int>(r->step_));
    c->init_from(*r, S(stream));
    auto h = new vkv_cache_s;
    h->impl = std::move(c);
    *out = h;
  });
}

int vkv_cache_inner_state(vkv_cache cache, vkv_array* arrays, int32_t* count) {
  return guard([&] {
    need(cache, "cache");
    need(arrays, "arrays");
    need(count, "count");
    if (auto* c = dynamic_cast<CompilableCache*>(cache->impl.get()))
      *count = c->inner_state(arrays);
    else if (auto* r = dynamic_cast<CompilableRotatingCache*>(cache->impl.get()))
      *count = r->inner_state(arrays);
    else if (auto* t = dynamic_cast<CompilableTurboQuantCache*>(cache->impl.get()))
      *count = t->inner_state(arrays);
    else
      throw Error("innerState is exposed for the fixed-buffer (compilable) caches only");
  });
}

static int dtype_bytes(int dt) {
  return dt == VKV_F32 || dt == VKV_U32 || dt == VKV_I32 ? 4 : dt == VKV_U8 || dt == VKV_BOOL ? 1 : 2;
}

static DynCopy dyn_args(const vkv_array& a, const vkv_array& b, const int32_t* start, int axis,
                        bool on_dst) {
  // a: the array the start applies to, b: the other side; shapes are b's
  if (a.ndim != b.ndim || a.ndim < 1 || a.ndim > 4) throw Error("arrays must have the same rank, 1 to 4");
  if (axis < 0) axis += a.ndim;
  if (axis < 0 || axis >= a.ndim) throw Error("axis out of range");
  if (dtype_bytes(a.dtype) != dtype_bytes(b.dtype)) throw Error("element sizes differ");
  for (int i = 0; i < a.ndim; i++)
    if (i != axis && a.shape[i] != b.shape[i]) throw Error("shapes differ outside the slice axis");
  if (b.shape[axis] > a.shape[axis]) throw Error("the slice is larger than the array along the axis");
  need(start, "start");
  DynCopy c{};
  const int pad = 4 - a.ndim;
  for (int i = 0; i < 4; i++) {
    const int j = i - pad;
    c.shape[i] = j < 0 ? 1 : b.shape[j];
    const int64_t as = j < 0 ? 0 : a.strides[j], bs = j < 0 ? 0 : b.strides[j];
    c.sstr[i] = on_dst ? bs : as;
    c.dstr[i] = on_dst ? as : bs;
  }
  c.src = static_cast<const uint8_t*>(on_dst ? b.data : a.data);
  c.dst = static_cast<uint8_t*>(on_dst ? a.data : b.data);
  c.axis = axis + pad;
  c.on_dst = on_dst ? 1 : 0;
  c.limit = a.shape[axis];
  c.start = start;
  return c;
}

int vkv_dynamic_slice_update(vkv_array* dst, const vkv_array* update, const int32_t* start, int32_t axis,
                             void* stream) {
  return guard([&] {
    need(dst, "dst");
    need(update, "update");
    const DynCopy c = dyn_args(*dst, *update, start, axis, true);
    if (c.shape[0] * c.shape[1] * c.shape[2] * c.shape[3] > 0) {
      need(dst->data, "dst data");
      need(update->data, "update data");
    }
    launch_dyn_copy(dtype_bytes(dst->dtype), c, S(stream));
  });
}

int vkv_dynamic_slice(const vkv_array* src, const int32_t* start, int32_t axis, vkv_array* out,
                      void* stream) {
  return guard([&] {
    need(src, "src");
    need(out, "out");
    const DynCopy c = dyn_args(*src, *out, start, axis, false);
    if (c.shape[0] * c.shape[1] * c.shape[2] * c.shape[3] > 0) {
      need(src->data, "src data");
      need(out->data, "out data");
    }
    launch_dyn_copy(dtype_bytes(src->dtype), c, S(stream));
  });
}

int vkv_cache_to_unquantized(vkv_cache quantized, void* stream, vkv_cache* out) {
  return guard([&] {
    need(quantized, "cache");
    need(out, "out");
    auto* q = dynamic_cast<QuantizedCache*>(quantized->impl.get());
    if (!q) throw Error("toUnquantized needs a QuantizedKVCache");
    auto h = new vkv_cache_s;
    try {
      h->impl = q->to_unquantized(S(stream));
    } catch (...) {
      delete h;
      throw;
    }
    *out = h;
  });
}

int vkv_cache_read_kv(vkv_cache cache, void* stream, vkv_array* keys, vkv_array* values) {
  return guard([&] {
    need(cache, "cache");
    need(keys, "keys");
    need(values, "values");
    cache->impl->read_kv(S(stream), keys, values);
  });
}

// -------------------------------------------------------------------- pool

int vkv_pool_create(const vkv_pool_params* params, vkv_pool* out) {
  return guard([&] {
    need(params, "params");
    need(out, "out");
    auto h = new vkv_pool_s;
    try {
      h->impl = std::make_unique<Pool>(*params);
    } catch (...) {
      delete h;
      throw;
    }
    *out = h;
  });
}

int vkv_pool_destroy(vkv_pool pool) {
  return guard([&] { delete pool; });
}

int vkv_pool_bytes(vkv_pool pool, int64_t* bytes) {
  return guard([&] {
    need(pool, "pool");
    need(bytes, "bytes");
    *bytes = static_cast<int64_t>(pool->impl->mem.size());
  });
}

int vkv_pool_view(vkv_pool pool, int32_t layer, const int32_t* block_table, int32_t table_stride,
                  const int32_t* seq_lens, int32_t n_seqs, int32_t max_len, vkv_paged_view* out) {
  return guard([&] {
    need(pool, "pool");
    need(out, "out");
    *out = pool->impl->view(layer, block_table, table_stride, seq_lens, n_seqs, max_len);
  });
}

int vkv_paged_append(vkv_pool pool, int32_t layer, const vkv_array* keys, const vkv_array* values,
                     const int32_t* slot_mapping, int64_t n_tokens, void* stream) {
  return guard([&] {
    need(pool, "pool");
    need(keys, "keys");
    pool->impl->append(layer, *keys, values, slot_mapping, n_tokens, S(stream));
  });
}

int vkv_paged_gather(const vkv_paged_view* kv, vkv_array* keys, vkv_array* values, void* stream) {
  return guard([&] {
    need(kv, "kv");
    vkv_array* outs[2] = {keys, values};
    KVSrc src = kvsrc_from_view(*kv);
    for (int which = 0; which < 2; which++) {
      vkv_array* o = outs[which];
      if (!o) continue;
      const int D = which ? kv->v_head_dim : kv->head_dim;
      if (o->ndim != 4 || !contiguous(*o) || o->dtype != kv->dtype || o->shape[0] != kv->n_seqs ||
          o->shape[1] != kv->n_kv_heads || o->shape[2] != kv->max_len || o->shape[3] != D)
        throw Error("gather output must be contiguous [n_seqs, Hkv, max_len, D] in the view dtype");
      GatherArgs g{};
      g.kv = src;
      g.n_seqs = kv->n_seqs;
      g.H = kv->n_kv_heads;
      g.T = kv->max_len;
      g.D = D;
      g.which = which;
      g.bits = kv->bits;
      g.group = kv->group_size;
      g.dtype = kv->dtype;
      g.out = o->data;
      launch_gather(g, 0, S(stream));
    }
  });
}

int vkv_paged_gather_quantized(const vkv_paged_view* kv, vkv_array* out, void* stream) {
  return guard([&] {
    need(kv, "kv");
    need(out, "out");
    if (kv->bits == 0) throw Error("code gather needs an affine view");
    const bool keys_only = (kv->flags & VKV_VIEW_KEYS_ONLY) != 0;
    KVSrc src = kvsrc_from_view(*kv);
    const int D = kv->head_dim;
    const int64_t W = static_cast<int64_t>(D) * kv->bits / 32, G = D / kv->group_size;
    for (int which = 0; which < (keys_only ? 1 : 2); which++) {
      vkv_array* o = out + 3 * which;
      for (int i = 0; i < 3; i++) {
        const int64_t last = i == 0 ? W : G;
        if (o[i].ndim != 4 || !contiguous(o[i]) || o[i].shape[0] != kv->n_seqs ||
            o[i].shape[1] != kv->n_kv_heads || o[i].shape[2] != kv->max_len || o[i].shape[3] != last)
          throw Error("code gather outputs must be contiguous reference-layout arrays");
      }
      GatherArgs g{};
      g.kv = src;
      g.n_seqs = kv->n_seqs;
      g.H = kv->n_kv_heads;
      g.T = kv->max_len;
      g.D = D;
      g.which = which;
      g.bits = kv->bits;
      g.group = kv->group_size;
      g.dtype = kv->dtype;
      g.out = o[0].data;
      g.out_s = o[1].data;
      g.out_b = o[2].data;
      launch_gather(g, 1, S(stream));
    }
  });
}

int vkv_pool_copy_blocks(vkv_pool pool, const int32_t* src, const int32_t* dst, int32_t n, void* stream) {
  return guard([&] {
    need(pool, "pool");
    if (n <= 0) return;
    need(src, "src");
    need(dst, "dst");
    Pool& p = *pool->impl;
    for (int i = 0; i < n; i++)
      if (src[i] < 0 || src[i] >= p.p.num_blocks || dst[i] < 0 || dst[i] >= p.p.num_blocks)
        throw Error("block id out of range");
    launch_copy_blocks(p.mem.bytes(), p.layer_bytes, p.p.n_layers, p.block_bytes, src, dst, n, S(stream));
  });
}

// ------------------------------------------------------------ prefix cache

int vkv_prefix_create(int32_t block_size, int32_t max_blocks, const char* model_key, vkv_pool pool,
                      vkv_prefix* out) {
  return guard([&] {
    need(out, "out");
    auto h = new vkv_prefix_s;
    try {
      h->impl = std::make_unique<PrefixManager>(block_size, max_blocks, model_key,
                                                pool ? pool->impl.get() : nullptr);
    } catch (...) {
      delete h;
      throw;
    }
    *out = h;
  });
}

int vkv_prefix_destroy(vkv_prefix mgr) {
  return guard([&] { delete mgr; });
}

int vkv_prefix_allocate(vkv_prefix mgr, int32_t* block) {
  return guard([&] {
    need(mgr, "mgr");
    need(block, "block");
    *block = mgr->impl->allocate();
  });
}

int vkv_prefix_free(vkv_prefix mgr, int32_t block) {
  return guard([&] {
    need(mgr, "mgr");
    mgr->impl->free_block(block);
  });
}

int vkv_prefix_release(vkv_prefix mgr, const int32_t* blocks, int32_t n) {
  return guard([&] {
    need(mgr, "mgr");
    if (n > 0) need(blocks, "blocks");
    for (int32_t i = n - 1; i >= 0; i--) mgr->impl->free_block(blocks[i]);
  });
}

int vkv_prefix_incref(vkv_prefix mgr, int32_t block) {
  return guard([&] {
    need(mgr, "mgr");
    mgr->impl->incref(block);
  });
}

int vkv_prefix_ref_count(vkv_prefix mgr, int32_t block, int32_t* ref_count) {
  return guard([&] {
    need(mgr, "mgr");
    need(ref_count, "ref_count");
    *ref_count = mgr->impl->ref_count(block);
  });
}

int vkv_prefix_find(vkv_prefix mgr, const char* hash, int32_t* block) {
  return guard([&] {
    need(mgr, "mgr");
    need(hash, "hash");
    need(block, "block");
    *block = mgr->impl->find(hash);
  });
}

int vkv_prefix_register(vkv_prefix mgr, int32_t block, const char* hash) {
  return guard([&] {
    need(mgr, "mgr");
    need(hash, "hash");
    mgr->impl->register_block(block, hash);
  });
}

int vkv_prefix_clear(vkv_prefix mgr) {
  return guard([&] {
    need(mgr, "mgr");
    mgr->impl->clear();
  });
}

int vkv_prefix_store(vkv_prefix mgr, const int64_t* tokens, int64_t n_tokens, const char* media_salt,
                     int32_t n_data_chunks, const int32_t* src_blocks, void* stream) {
  return guard([&] {
    need(mgr, "mgr");
    if (n_tokens > 0) need(tokens, "tokens");
    mgr->impl->store(tokens, n_tokens, media_salt, n_data_chunks, src_blocks, S(stream));
  });
}

int vkv_prefix_fetch(vkv_prefix mgr, const int64_t* tokens, int64_t n_tokens, const char* media_salt,
                     int32_t* blocks, int32_t capacity, int32_t* n_blocks, int64_t* matched_tokens) {
  return guard([&] {
    need(mgr, "mgr");
    need(n_blocks, "n_blocks");
    need(matched_tokens, "matched_tokens");
    if (capacity > 0) need(blocks, "blocks");
    if (n_tokens > 0) need(tokens, "tokens");
    mgr->impl->fetch(tokens, n_tokens, media_salt, blocks, capacity, n_blocks, matched_tokens);
  });
}

int vkv_prefix_writable(vkv_prefix mgr, int32_t block, void* stream, int32_t* out_block) {
  return guard([&] {
    need(mgr, "mgr");
    need(out_block, "out_block");
    *out_block = mgr->impl->writable(block, S(stream));
  });
}

int vkv_prefix_stats_get(vkv_prefix mgr, vkv_prefix_stats* out) {
  return guard([&] {
    need(mgr, "mgr");
    need(out, "out");
    *out = mgr->impl->stats();
  });
}

int vkv_prefix_block_tokens(vkv_prefix mgr, int32_t block, int32_t* n_tokens) {
  return guard([&] {
    need(mgr, "mgr");
    need(n_tokens, "n_tokens");
    *n_tokens = mgr->impl->block_tokens(block);
  });
}

int vkv_block_hash(const char* parent_hash, const int64_t* tokens, int64_t n_tokens,
                   const char* model_key, const char* media_salt, char* out) {
  return guard([&] {
    need(out, "out");
    if (n_tokens > 0) need(tokens, "tokens");
    std::string p = parent_hash ? parent_hash : "", k = model_key ? model_key : "",
                s = media_salt ? media_salt : "";
    std::string h = PrefixManager::block_hash(parent_hash ? &p : nullptr, tokens, n_tokens,
                                              model_key ? &k : nullptr, media_salt ? &s : nullptr);
    memcpy(out, h.c_str(), 65);
  });
}

int vkv_array_copy(const vkv_array* src, vkv_array* dst, void* stream) {
  return guard([&] {
    need(src, "src");
    need(dst, "dst");
    if (src->ndim != dst->ndim || src->ndim < 1 || src->ndim > 4) throw Error("copy needs equal ranks 1..4");
    for (int i = 0; i < src->ndim; i++)
      if (src->shape[i] != dst->shape[i]) throw Error("copy needs equal shapes");
    auto esz = [](int dt) { return dt == VKV_F32 || dt == VKV_U32 || dt == VKV_I32 ? 4 : dt == VKV_U8 || dt == VKV_BOOL ? 1 : 2; };
    if (esz(src->dtype) != esz(dst->dtype)) throw Error("copy needs equal element sizes");
    int64_t n[4] = {1, 1, 1, 1}, ss[4] = {0, 0, 0, 0}, ds[4] = {0, 0, 0, 0};
    for (int i = 0; i < src->ndim; i++) {
      n[4 - src->ndim + i] = src->shape[i];
      ss[4 - src->ndim + i] = src->strides[i];
      ds[4 - src->ndim + i] = dst->strides[i];
    }
    launch_copy4d(esz(src->dtype), src->data, n, ss, dst->data, ds, S(stream));
  });
}

// ----------------------------------------------------------- kernel timing

int vkv_kernel_timing(int32_t enable) {
  return guard([&] { timing_enable(enable != 0); });
}

int vkv_kernel_timing_read(int32_t kind, double* total_ms, int32_t* count) {
  return guard([&] {
    need(total_ms, "total_ms");
    need(count, "count");
    if (kind < 0 || kind >= kTimeKinds) throw Error("unknown timing kind");
    int c = 0;
    timing_read(kind, total_ms, &c);
    *count = c;
  });
}

// --------------------------------------------------------------- synthetic

int vkv_fill_normal(void* data, int32_t dtype, int64_t n, uint64_t seed, float std, void* stream) {
  return guard([&] {
    if (n > 0) need(data, "data");
    if (!is_float(dtype)) throw Error("dtype must be f32, f16 or bf16");
    launch_fill_normal(dtype, data, n, seed, std, S(stream));
  });
}

}  // extern "C"
