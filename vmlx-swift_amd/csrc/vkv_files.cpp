// vkv_files.cpp -- on-disk cache formats, read and written straight from
// the library's device caches and pool blocks:
//   * the prompt-cache safetensors file of savePromptCache / loadPromptCache
//     (Libraries/MLXLMCommon/KVCache.swift:1613-1845): tensors "i.j" (state
//     array j of layer i), metadata "0.i.j" (metaState), "1.<key>" (user
//     metadata), "2.i" (class name);
//   * the disk tier's version-2 record (Cache/TQDiskSerializer.swift:15-103,
//     :240-330, :455-510, :800-830) for the standard, rotating and
//     quantized attention layers, keyed by DiskCache.hashTokens
//     (Cache/DiskCache.swift:659-682);
//   * a prompt-cache file written from / read into a sequence's paged pool
//     blocks, with no intermediate cache object.
// The safetensors container (8-byte little-endian header length, a JSON
// header of {name: {dtype, shape, data_offsets}} plus "__metadata__", then
// the data) is written and parsed here; the parser validates every offset
// against the file before any device memory is touched.
#include <string.h>

#include <algorithm>
#include <cstdio>
#include <fstream>
#include <functional>
#include <map>
#include <string>
#include <vector>

#include "sha256.h"
#include "vkv_host.h"

using namespace vkv;

namespace {

// ------------------------------------------------------------------ JSON

struct JVal {
  enum Kind { Null, Bool, Int, Str, Arr, Obj } kind = Null;
  bool b = false;
  int64_t i = 0;
  std::string s;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal* get(const std::string& k) const {
    for (auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

class JParser {
 public:
  JParser(const char* p, size_t n) : p_(p), e_(p + n) {}
  JVal parse() {
    JVal v = value(0);
    ws();
    if (p_ != e_) fail("trailing characters");
    return v;
  }

 private:
  const char *p_, *e_;
  [[noreturn]] void fail(const char* m) {
    throw Error(std::string("safetensors header: ") + m);
  }
  void ws() {
    while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
  }
  void expect(char c) {
    ws();
    if (p_ >= e_ || *p_ != c) fail("unexpected character");
    p_++;
  }
  static void put_utf8(std::string& o, uint32_t cp) {
    if (cp < 0x80) {
      o += static_cast<char>(cp);
    } else if (cp < 0x800) {
      o += static_cast<char>(0xC0 | (cp >> 6));
      o += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      o += static_cast<char>(0xE0 | (cp >> 12));
      o += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      o += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
      o += static_cast<char>(0xF0 | (cp >> 18));
      o += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
      o += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      o += static_cast<char>(0x80 | (cp & 0x3F));
    }
  }
  uint32_t hex4() {
    if (e_ - p_ < 4) fail("short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; k++) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
      else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
      else fail("bad \\u escape");
    }
    return v;
  }
  std::string str() {
    expect('"');
    std::string o;
    while (true) {
      if (p_ >= e_) fail("unterminated string");
      const char c = *p_++;
      if (c == '"') break;
      if (c != '\\') {
        o += c;
        continue;
      }
      if (p_ >= e_) fail("unterminated escape");
      const char x = *p_++;
      switch (x) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            if (e_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') fail("lone surrogate");
            p_ += 2;
            const uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(o, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
    return o;
  }
  JVal value(int depth) {
    if (depth > 16) fail("nesting too deep");
    ws();
    if (p_ >= e_) fail("unexpected end");
    JVal v;
    const char c = *p_;
    if (c == '{') {
      v.kind = JVal::Obj;
      p_++;
      ws();
      if (p_ < e_ && *p_ == '}') {
        p_++;
        return v;
      }
      while (true) {
        std::string k = str();
        expect(':');
        v.obj.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (p_ < e_ && *p_ == ',') {
          p_++;
          continue;
        }
        expect('}');
        return v;
      }
    }
    if (c == '[') {
      v.kind = JVal::Arr;
      p_++;
      ws();
      if (p_ < e_ && *p_ == ']') {
        p_++;
        return v;
      }
      while (true) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (p_ < e_ && *p_ == ',') {
          p_++;
          continue;
        }
        expect(']');
        return v;
      }
    }
    if (c == '"') {
      v.kind = JVal::Str;
      v.s = str();
      return v;
    }
    if (c == '-' || (c >= '0' && c <= '9')) {
      v.kind = JVal::Int;
      bool neg = false;
      if (*p_ == '-') {
        neg = true;
        p_++;
      }
      if (p_ >= e_ || *p_ < '0' || *p_ > '9') fail("bad number");
      int64_t x = 0;
      while (p_ < e_ && *p_ >= '0' && *p_ <= '9') {
        if (x > (INT64_MAX - 9) / 10) fail("number too large");
        x = x * 10 + (*p_++ - '0');
      }
      if (p_ < e_ && (*p_ == '.' || *p_ == 'e' || *p_ == 'E')) fail("non-integer number");
      v.i = neg ? -x : x;
      return v;
    }
    auto word = [&](const char* w) {
      const size_t n = strlen(w);
      if (static_cast<size_t>(e_ - p_) < n || strncmp(p_, w, n) != 0) fail("bad literal");
      p_ += n;
    };
    if (c == 't') {
      word("true");
      v.kind = JVal::Bool;
      v.b = true;
      return v;
    }
    if (c == 'f') {
      word("false");
      v.kind = JVal::Bool;
      return v;
    }
    if (c == 'n') {
      word("null");
      return v;
    }
    fail("unexpected character");
  }
};

std::string jstr(const std::string& s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      default:
        if (c < 0x20) {
          char b[8];
          snprintf(b, sizeof(b), "\\u%04x", c);
          o += b;
        } else {
          o += static_cast<char>(c);
        }
    }
  }
  return o + "\"";
}

// ----------------------------------------------------------- safetensors

const char* st_dtype(int dt) {
  switch (dt) {
    case VKV_F32: return "F32";
    case VKV_F16: return "F16";
    case VKV_BF16: return "BF16";
    case VKV_U32: return "U32";
    case VKV_I32: return "I32";
    case VKV_U8: return "U8";
    case VKV_BOOL: return "BOOL";
  }
  throw Error("no safetensors dtype for this array");
}

int st_dtype_code(const std::string& s) {
  if (s == "F32") return VKV_F32;
  if (s == "F16") return VKV_F16;
  if (s == "BF16") return VKV_BF16;
  if (s == "U32") return VKV_U32;
  if (s == "I32") return VKV_I32;
  if (s == "U8") return VKV_U8;
  if (s == "BOOL") return VKV_BOOL;
  return -1;
}

int dt_bytes(int dt) {
  return dt == VKV_F32 || dt == VKV_U32 || dt == VKV_I32 ? 4 : dt == VKV_U8 || dt == VKV_BOOL ? 1 : 2;
}

struct HostTensor {
  int dtype = VKV_F32;
  std::vector<int64_t> shape;
  std::vector<uint8_t> data;
};

using TensorMap = std::map<std::string, HostTensor>;          // sorted: deterministic files
using StrMap = std::map<std::string, std::string>;

void write_safetensors(const std::string& path, const TensorMap& ts, const StrMap& meta) {
  std::string h = "{\"__metadata__\":{";
  bool first = true;
  for (auto& kv : meta) {
    if (!first) h += ",";
    first = false;
    h += jstr(kv.first) + ":" + jstr(kv.second);
  }
  h += "}";
  int64_t off = 0;
  for (auto& kv : ts) {
    const HostTensor& t = kv.second;
    h += "," + jstr(kv.first) + ":{\"dtype\":\"" + st_dtype(t.dtype) + "\",\"shape\":[";
    for (size_t i = 0; i < t.shape.size(); i++) h += (i ? "," : "") + std::to_string(t.shape[i]);
    const int64_t n = static_cast<int64_t>(t.data.size());
    h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + n) + "]}";
    off += n;
  }
  h += "}";
  while ((8 + h.size()) % 8) h += ' ';  // the data starts 8-byte aligned
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  if (!f) throw Error("cannot open " + path + " for writing");
  uint8_t len[8];
  const uint64_t hl = h.size();
  for (int i = 0; i < 8; i++) len[i] = static_cast<uint8_t>(hl >> (8 * i));
  f.write(reinterpret_cast<const char*>(len), 8);
  f.write(h.data(), static_cast<std::streamsize>(h.size()));
  for (auto& kv : ts)
    f.write(reinterpret_cast<const char*>(kv.second.data.data()),
            static_cast<std::streamsize>(kv.second.data.size()));
  if (!f) throw Error("write to " + path + " failed");
}

struct StEntry {
  int dtype;
  std::vector<int64_t> shape;
  int64_t begin, end;
};

struct StFile {
  std::string path;
  int64_t data_start = 0;
  std::map<std::string, StEntry> tensors;
  StrMap meta;
};

// Parses and validates the header; no tensor data is read.
StFile read_safetensors_header(const std::string& path) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) throw Error("cannot open " + path);
  const int64_t size = static_cast<int64_t>(f.tellg());
  if (size < 8) throw Error(path + ": not a safetensors file (too short)");
  f.seekg(0);
  uint8_t len[8];
  f.read(reinterpret_cast<char*>(len), 8);
  uint64_t hl = 0;
  for (int i = 0; i < 8; i++) hl |= static_cast<uint64_t>(len[i]) << (8 * i);
  if (hl == 0 || hl > static_cast<uint64_t>(size - 8) || hl > (uint64_t{100} << 20))
    throw Error(path + ": bad safetensors header length");
  std::string h(hl, '\0');
  f.read(&h[0], static_cast<std::streamsize>(hl));
  if (!f) throw Error(path + ": short read of the header");
  JVal root = JParser(h.data(), h.size()).parse();
  if (root.kind != JVal::Obj) throw Error(path + ": the header is not a JSON object");
  StFile out;
  out.path = path;
  out.data_start = 8 + static_cast<int64_t>(hl);
  const int64_t data_len = size - out.data_start;
  for (auto& kv : root.obj) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != JVal::Obj) throw Error(path + ": __metadata__ is not an object");
      for (auto& m : kv.second.obj) {
        if (m.second.kind != JVal::Str) throw Error(path + ": metadata values must be strings");
        out.meta[m.first] = m.second.s;
      }
      continue;
    }
    const JVal& t = kv.second;
    const JVal *dt = t.get("dtype"), *sh = t.get("shape"), *of = t.get("data_offsets");
    if (t.kind != JVal::Obj || !dt || !sh || !of || dt->kind != JVal::Str || sh->kind != JVal::Arr ||
        of->kind != JVal::Arr || of->arr.size() != 2)
      throw Error(path + ": malformed entry for tensor " + kv.first);
    StEntry e;
    e.dtype = st_dtype_code(dt->s);
    if (e.dtype < 0) throw Error(path + ": unsupported dtype " + dt->s + " for tensor " + kv.first);
    int64_t n = 1;
    for (auto& d : sh->arr) {
      if (d.kind != JVal::Int || d.i < 0 || d.i > (int64_t{1} << 40))
        throw Error(path + ": bad shape for tensor " + kv.first);
      e.shape.push_back(d.i);
      // the element count stays below 2^42, checked before the product
      // could overflow
      constexpr int64_t kMaxElems = int64_t{1} << 42;
      if (d.i != 0 && n > kMaxElems / d.i) throw Error(path + ": tensor " + kv.first + " is too large");
      n *= d.i;
    }
    if (of->arr[0].kind != JVal::Int || of->arr[1].kind != JVal::Int)
      throw Error(path + ": bad data_offsets for tensor " + kv.first);
    e.begin = of->arr[0].i;
    e.end = of->arr[1].i;
    if (e.begin < 0 || e.end < e.begin || e.end > data_len || e.end - e.begin != n * dt_bytes(e.dtype))
      throw Error(path + ": data_offsets of tensor " + kv.first + " do not fit its shape or the file");
    out.tensors[kv.first] = e;
  }
  return out;
}

HostTensor read_tensor(const StFile& f, const std::string& name) {
  auto it = f.tensors.find(name);
  if (it == f.tensors.end()) throw Error(f.path + ": no tensor " + name);
  const StEntry& e = it->second;
  std::ifstream in(f.path, std::ios::binary);
  if (!in) throw Error("cannot open " + f.path);
  in.seekg(f.data_start + e.begin);
  HostTensor t;
  t.dtype = e.dtype;
  t.shape = e.shape;
  t.data.resize(static_cast<size_t>(e.end - e.begin));
  if (!t.data.empty()) in.read(reinterpret_cast<char*>(t.data.data()), static_cast<std::streamsize>(t.data.size()));
  if (!in) throw Error(f.path + ": short read of tensor " + name);
  return t;
}

// ----------------------------------------------------- device <-> host

int64_t numel(const vkv_array& a) {
  int64_t n = 1;
  for (int i = 0; i < a.ndim; i++) n *= a.shape[i];
  return n;
}

// A device array (any strides, up to 4 dims) as a contiguous host tensor.
HostTensor to_host(const vkv_array& a, hipStream_t st) {
  HostTensor t;
  t.dtype = a.dtype;
  for (int i = 0; i < a.ndim; i++) t.shape.push_back(a.shape[i]);
  const int es = dt_bytes(a.dtype);
  const int64_t n = numel(a);
  t.data.resize(static_cast<size_t>(n * es));
  if (n == 0) return t;
  bool contiguous = true;
  int64_t s = 1;
  for (int i = a.ndim - 1; i >= 0; i--) {
    if (a.shape[i] != 1 && a.strides[i] != s) contiguous = false;
    s *= a.shape[i];
  }
  if (contiguous) {
    VKV_HIP(hipMemcpyAsync(t.data.data(), a.data, t.data.size(), hipMemcpyDeviceToHost, st));
    VKV_HIP(hipStreamSynchronize(st));
    return t;
  }
  if (es != 2 && es != 4) throw Error("strided byte arrays are not supported here");
  DevBuf tmp(t.data.size());
  int64_t sh[4] = {1, 1, 1, 1}, ss[4] = {0, 0, 0, 0}, ds[4];
  for (int i = 0; i < a.ndim; i++) {
    sh[4 - a.ndim + i] = a.shape[i];
    ss[4 - a.ndim + i] = a.strides[i];
  }
  ds[3] = 1;
  ds[2] = sh[3];
  ds[1] = sh[2] * sh[3];
  ds[0] = sh[1] * sh[2] * sh[3];
  launch_copy4d(es, a.data, sh, ss, tmp.get(), ds, st);
  VKV_HIP(hipMemcpyAsync(t.data.data(), tmp.get(), t.data.size(), hipMemcpyDeviceToHost, st));
  VKV_HIP(hipStreamSynchronize(st));
  return t;
}

// A host tensor copied into a new device buffer; `a` describes it.
DevBuf to_device(const HostTensor& t, hipStream_t st, vkv_array* a) {
  if (t.shape.size() > 4) throw Error("arrays of more than 4 dims are not supported here");
  DevBuf b(std::max<size_t>(t.data.size(), 1));
  if (!t.data.empty()) {
    VKV_HIP(hipMemcpyAsync(b.get(), t.data.data(), t.data.size(), hipMemcpyHostToDevice, st));
    VKV_HIP(hipStreamSynchronize(st));
  }
  *a = vkv_array{};
  a->data = b.get();
  a->dtype = t.dtype;
  a->ndim = static_cast<int32_t>(t.shape.size());
  int64_t s = 1;
  for (int i = a->ndim - 1; i >= 0; i--) {
    a->shape[i] = t.shape[i];
    a->strides[i] = s;
    s *= t.shape[i];
  }
  return b;
}

HostTensor int32_vec(const std::vector<int32_t>& v) {
  HostTensor t;
  t.dtype = VKV_I32;
  t.shape = {static_cast<int64_t>(v.size())};
  t.data.resize(v.size() * 4);
  memcpy(t.data.data(), v.data(), t.data.size());
  return t;
}

// readMetaInt32 (TQDiskSerializer.swift:168-176): a 1-element int32 array
// (or a 0-dim one), else "absent".
bool meta_int32(const StFile& f, const std::string& key, int32_t* out) {
  auto it = f.tensors.find(key);
  if (it == f.tensors.end() || it->second.dtype != VKV_I32) return false;
  const auto& sh = it->second.shape;
  if (!(sh.empty() || (sh.size() == 1 && sh[0] == 1))) return false;
  HostTensor t = read_tensor(f, key);
  memcpy(out, t.data.data(), 4);
  return true;
}

// ------------------------------------------------------- cache objects

const char* class_name(int kind) {
  switch (kind) {
    case VKV_CACHE_ROTATING:
    case VKV_CACHE_COMPILABLE_ROTATING: return "RotatingKVCache";
    case VKV_CACHE_QUANTIZED: return "QuantizedKVCache";
    case VKV_CACHE_TURBOQUANT:
    case VKV_CACHE_COMPILABLE_TURBOQUANT: return "TurboQuantKVCache";  // not loadable, as in the reference
    default: return "KVCache";  // KVCacheSimple and the fixed-buffer cache
  }
}

int parse_int(const std::string& s, int fallback) {
  char* end = nullptr;
  const long v = strtol(s.c_str(), &end, 10);
  return (end && *end == '\0' && !s.empty()) ? static_cast<int>(v) : fallback;
}

// A cache of the class, built from its metaState before the state is set
// (loadPromptCache, KVCache.swift:1715-1760).
std::unique_ptr<Cache> new_cache_for(const std::string& cls, const std::vector<std::string>& info) {
  vkv_cache_params p{};
  if (cls == "KVCache" || cls == "KVCacheSimple") {
    p.kind = VKV_CACHE_SIMPLE;
  } else if (cls == "RotatingKVCache") {
    if (info.size() < 5) throw Error("Invalid RotatingKVCache metaState - expected 5 values");
    if (info[1] == "None")
      throw Error("RotatingKVCache with maxSize=None is not supported. This cache was created "
                  "with invalid parameters.");
    const int m = parse_int(info[1], -1);
    if (m <= 0) throw Error("Failed to parse RotatingKVCache maxSize from: " + info[1]);
    p.kind = VKV_CACHE_ROTATING;
    p.max_size = m;
  } else if (cls == "QuantizedKVCache") {
    // the reference builds QuantizedKVCache() (group 64, bits 8) and sets
    // only the offset from metaState; the group size and bits it saved
    // (metaState [step, offset, groupSize, bits], :1168-1177) are used here
    // so a 4-bit cache comes back as one
    p.kind = VKV_CACHE_QUANTIZED;
    p.step = info.size() >= 1 ? parse_int(info[0], 256) : 256;
    p.group_size = info.size() >= 3 ? parse_int(info[2], 64) : 64;
    p.bits = info.size() >= 4 ? parse_int(info[3], 8) : 8;
  } else {
    throw Error("Unknown cache class: " + cls);
  }
  return make_cache(p);
}

// Sets a cache's state from host tensors (device copies made and released
// here: the caches copy state in).
void set_state_from_host(Cache& c, const std::vector<HostTensor>& arrays, hipStream_t st) {
  std::vector<DevBuf> bufs;
  std::vector<vkv_array> descs(arrays.size());
  for (size_t j = 0; j < arrays.size(); j++) bufs.push_back(to_device(arrays[j], st, &descs[j]));
  c.set_state(descs.data(), static_cast<int>(descs.size()), st);
  VKV_HIP(hipStreamSynchronize(st));
}

std::vector<HostTensor> state_to_host(Cache& c, hipStream_t st) {
  vkv_array s[6];
  const int n = c.state(st, s);
  std::vector<HostTensor> out;
  for (int j = 0; j < n; j++) out.push_back(to_host(s[j], st));
  return out;
}

// DiskCache.hashTokens (DiskCache.swift:659-682): SHA-256 of the model key,
// "|media:" + salt, then the tokens as raw little-endian Int64; the first 32
// hex digits.
std::string disk_hash(const int64_t* tokens, int64_t n, const char* model_key, const char* salt) {
  Sha256 h;
  if (model_key) h.update(model_key, strlen(model_key));
  if (salt) {
    static const char tag[] = "|media:";
    h.update(tag, sizeof(tag) - 1);
    h.update(salt, strlen(salt));
  }
  if (n > 0) h.update(tokens, static_cast<size_t>(n) * sizeof(int64_t));
  return h.hex_digest().substr(0, 32);
}

void put_meta_out(const StrMap& m, char* buf, int64_t len, int32_t* count) {
  int64_t need = 0;
  for (auto& kv : m) need += static_cast<int64_t>(kv.first.size() + kv.second.size()) + 2;
  if (count) *count = static_cast<int32_t>(m.size());
  if (!buf) return;
  if (need > len) throw Error("metadata buffer too small (" + std::to_string(need) + " bytes needed)");
  char* p = buf;
  for (auto& kv : m) {
    memcpy(p, kv.first.c_str(), kv.first.size() + 1);
    p += kv.first.size() + 1;
    memcpy(p, kv.second.c_str(), kv.second.size() + 1);
    p += kv.second.size() + 1;
  }
}

}  // namespace

// ------------------------------------------------------------ the C ABI

namespace {
// The C ABI's error convention (vkv_capi.cpp): 0, or 1 with the message
// kept for vkv_last_error().
template <class F>
int guarded(F&& f) {
  return guarded_call(std::function<void()>(f));
}
}  // namespace

extern "C" {

int vkv_prompt_cache_save(const char* path, const vkv_cache* caches, int32_t n_caches,
                          const char* const* meta_keys, const char* const* meta_values,
                          int32_t n_meta, void* stream) {
  return guarded([&] {
    if (!path) throw Error("path is NULL");
    if (n_caches < 0 || (n_caches > 0 && !caches)) throw Error("caches is NULL");
    if (n_meta > 0 && (!meta_keys || !meta_values)) throw Error("metadata is NULL");
    const hipStream_t st = S(stream);
    TensorMap ts;
    StrMap meta;
    for (int i = 0; i < n_caches; i++) {
      if (!caches[i]) throw Error("cache " + std::to_string(i) + " is NULL");
      Cache& c = *caches[i]->impl;
      auto arrays = state_to_host(c, st);
      for (size_t j = 0; j < arrays.size(); j++)
        ts[std::to_string(i) + "." + std::to_string(j)] = std::move(arrays[j]);
      auto info = c.meta_state();
      for (size_t j = 0; j < info.size(); j++)
        meta["0." + std::to_string(i) + "." + std::to_string(j)] = info[j];
      meta["2." + std::to_string(i)] = class_name(c.kind());
    }
    for (int k = 0; k < n_meta; k++) {
      if (!meta_keys[k] || !meta_values[k]) throw Error("metadata entry is NULL");
      meta[std::string("1.") + meta_keys[k]] = meta_values[k];
    }
    write_safetensors(path, ts, meta);
  });
}

int vkv_prompt_cache_load(const char* path, void* stream, vkv_cache* caches, int32_t capacity,
                          int32_t* n_caches, char* meta_buf, int64_t meta_buf_len,
                          int32_t* n_meta) {
  return guarded([&] {
    if (!path) throw Error("path is NULL");
    if (!n_caches) throw Error("n_caches is NULL");
    const hipStream_t st = S(stream);
    StFile f = read_safetensors_header(path);
    // unflattenArrays / unflattenMetadata (KVCache.swift:1790-1845)
    std::map<int, std::map<int, std::string>> arr_keys;
    for (auto& kv : f.tensors) {
      const auto dot = kv.first.find('.');
      if (dot == std::string::npos) continue;
      const int i = parse_int(kv.first.substr(0, dot), -1);
      const int j = parse_int(kv.first.substr(dot + 1), -1);
      if (i >= 0 && j >= 0) arr_keys[i][j] = kv.first;
    }
    std::map<int, std::map<int, std::string>> info_map;
    std::map<int, std::string> classes;
    StrMap user;
    for (auto& kv : f.meta) {
      const std::string& k = kv.first;
      if (k.rfind("0.", 0) == 0) {
        const auto d2 = k.find('.', 2);
        if (d2 == std::string::npos) continue;
        const int i = parse_int(k.substr(2, d2 - 2), -1), j = parse_int(k.substr(d2 + 1), -1);
        if (i >= 0 && j >= 0) info_map[i][j] = kv.second;
      } else if (k.rfind("1.", 0) == 0) {
        user[k.substr(2)] = kv.second;
      } else if (k.rfind("2.", 0) == 0) {
        const int i = parse_int(k.substr(2), -1);
        if (i >= 0) classes[i] = kv.second;
      }
    }
    if (classes.empty() && info_map.empty() && arr_keys.empty())
      throw Error("Invalid cache metadata format");
    const int n_data = arr_keys.empty() ? 0 : arr_keys.rbegin()->first + 1;
    const int n_info = info_map.empty() ? 0 : info_map.rbegin()->first + 1;
    const int n_cls = classes.empty() ? 0 : classes.rbegin()->first + 1;
    if (n_data != n_info || n_data != n_cls) throw Error("Mismatch in cache counts");
    // validate every layer's class and metaState before building any cache
    // (constructing a cache object allocates no device memory)
    std::vector<std::vector<std::string>> infos(n_data);
    for (int i = 0; i < n_data; i++) {
      auto& m = info_map[i];
      const int nj = m.empty() ? 0 : m.rbegin()->first + 1;
      infos[i].assign(nj, "");
      for (auto& kv : m) infos[i][kv.first] = kv.second;
      if (!classes.count(i)) throw Error("Unknown cache class: ");
      new_cache_for(classes[i], infos[i]);  // throws on an unknown class or bad metaState
    }
    *n_caches = n_data;
    put_meta_out(user, meta_buf, meta_buf_len, n_meta);
    if (!caches) return;  // counting call
    if (capacity < n_data) throw Error("caches capacity is smaller than the file's layer count");
    std::vector<std::unique_ptr<Cache>> built;
    for (int i = 0; i < n_data; i++) {
      auto c = new_cache_for(classes[i], infos[i]);
      std::vector<HostTensor> arrays;
      auto& am = arr_keys[i];
      const int nj = am.empty() ? 0 : am.rbegin()->first + 1;
      for (int j = 0; j < nj; j++)
        if (am.count(j)) arrays.push_back(read_tensor(f, am[j]));
      if (!arrays.empty()) set_state_from_host(*c, arrays, st);
      if (!infos[i].empty()) c->set_meta_state(infos[i]);
      built.push_back(std::move(c));
    }
    for (int i = 0; i < n_data; i++) {
      auto h = new vkv_cache_s;
      h->impl = std::move(built[i]);
      caches[i] = h;
    }
  });
}

int vkv_disk_hash_tokens(const int64_t* tokens, int64_t n_tokens, const char* model_key,
                         const char* media_salt, char* out) {
  return guarded([&] {
    if (!out) throw Error("out is NULL");
    if (n_tokens > 0 && !tokens) throw Error("tokens is NULL");
    const std::string h = disk_hash(tokens, n_tokens, model_key, media_salt);
    memcpy(out, h.c_str(), 33);
  });
}

namespace {

// serializeTQLayer (TQDiskSerializer.swift:368-429): the encoded records
// (tq_i_ck_* / tq_i_cv_*, shapes, index bits, seeds), the offset and, when
// tokens follow the encoded ones, the exact window (tq_i_window_*).
void save_tq_layer(TurboQuantCache& t, const std::string& I, TensorMap& ts, hipStream_t st) {
  vkv_tq_encoded ek, ev;
  t.encoded(&ek, &ev);
  const std::string k = "tq_" + I + "_ck_", v = "tq_" + I + "_cv_";
  ts[k + "indices"] = to_host(ek.indices, st);
  ts[k + "qjl"] = to_host(ek.qjl, st);
  ts[k + "res_norms"] = to_host(ek.res_norms, st);
  ts[k + "vec_norms"] = to_host(ek.vec_norms, st);
  if (ek.sink.ndim) ts[k + "sink"] = to_host(ek.sink, st);
  if (ek.tail.ndim) ts[k + "tail"] = to_host(ek.tail, st);
  ts["__tq_" + I + "_ck_shape__"] = int32_vec({ek.shape[0], ek.shape[1], ek.shape[2], ek.shape[3]});
  ts["__tq_" + I + "_ck_index_bits__"] = int32_vec({ek.index_bits});
  ts["__tq_" + I + "_ck_seed__"] = int32_vec({ek.seed});
  ts[v + "indices"] = to_host(ev.indices, st);
  ts[v + "norms"] = to_host(ev.vec_norms, st);
  if (ev.sink.ndim) ts[v + "sink"] = to_host(ev.sink, st);
  if (ev.tail.ndim) ts[v + "tail"] = to_host(ev.tail, st);
  ts["__tq_" + I + "_cv_shape__"] = int32_vec({ev.shape[0], ev.shape[1], ev.shape[2], ev.shape[3]});
  ts["__tq_" + I + "_cv_index_bits__"] = int32_vec({ev.index_bits});
  ts["__tq_" + I + "_cv_seed__"] = int32_vec({ev.seed});
  ts["__tq_" + I + "_offset__"] = int32_vec({static_cast<int32_t>(t.offset)});
  const int64_t encoded = static_cast<int64_t>(ek.shape[2]) + (ek.sink.ndim ? ek.sink.shape[2] : 0) +
                          (ek.tail.ndim ? ek.tail.shape[2] : 0);
  const int64_t live = t.offset - encoded;
  vkv_array wk{}, wv{};
  if (live > 0 && t.window_state(&wk, &wv)) {
    if (wk.shape[2] != live || wv.shape[2] != live) return;
    ts["tq_" + I + "_window_keys"] = to_host(wk, st);
    ts["tq_" + I + "_window_values"] = to_host(wv, st);
  }
}

// deserializeTQLayer (TQDiskSerializer.swift:1244-1346) checks: every
// record field present, the counts of encoded key and value tokens equal
// and positive, the offset (default: the key shape's token count) not below
// them, and exactly offset - count window tokens when that is positive.
// Returns the offset.
int64_t check_tq_layer(const StFile& f, const std::string& I) {
  auto has = [&](const std::string& k) { return f.tensors.count(k) > 0; };
  const std::string k = "tq_" + I + "_ck_", v = "tq_" + I + "_cv_";
  int32_t x = 0;
  for (const char* n : {"indices", "qjl", "res_norms", "vec_norms"})
    if (!has(k + n)) throw Error("layer " + I + ": incomplete TurboQuant payload: required miss");
  if (!has(v + "indices") || !has(v + "norms"))
    throw Error("layer " + I + ": incomplete TurboQuant payload: required miss");
  for (const char* n : {"ck", "cv"}) {
    const std::string p = "__tq_" + I + "_" + n;
    if (!has(p + "_shape__") || !meta_int32(f, p + "_index_bits__", &x) ||
        !meta_int32(f, p + "_seed__", &x))
      throw Error("layer " + I + ": incomplete TurboQuant payload: required miss");
  }
  auto shape = [&](const std::string& key) {
    HostTensor t = read_tensor(f, key);
    if (t.dtype != VKV_I32 || t.shape.size() != 1) throw Error("layer " + I + ": bad TurboQuant shape");
    std::vector<int32_t> out(t.shape[0]);
    memcpy(out.data(), t.data.data(), out.size() * 4);
    return out;
  };
  auto count = [&](const std::vector<int32_t>& sh, const std::string& pre) {
    if (sh.size() < 3) return int64_t{0};
    int64_t n = sh[2];
    for (const char* part : {"sink", "tail"}) {
      auto it = f.tensors.find(pre + part);
      if (it != f.tensors.end() && it->second.shape.size() == 4) n += it->second.shape[2];
    }
    return n;
  };
  const auto ks = shape("__tq_" + I + "_ck_shape__"), vs = shape("__tq_" + I + "_cv_shape__");
  const int64_t nk = count(ks, k), nv = count(vs, v);
  int64_t offset = ks.size() >= 3 ? ks[2] : 0;
  if (has("__tq_" + I + "_offset__")) {
    if (!meta_int32(f, "__tq_" + I + "_offset__", &x)) throw Error("layer " + I + ": bad TurboQuant offset");
    offset = x;
  }
  if (nk <= 0 || nk != nv || offset < nk)
    throw Error("layer " + I + ": inconsistent TurboQuant token counts: required miss");
  const int64_t window = offset - nk;
  const bool wk = has("tq_" + I + "_window_keys"), wv = has("tq_" + I + "_window_values");
  if (window == 0 && (wk || wv))
    throw Error("layer " + I + ": unexpected TurboQuant window: required miss");
  if (window > 0) {
    if (!wk || !wv) throw Error("layer " + I + ": missing TurboQuant window: required miss");
    const auto& a = f.tensors.at("tq_" + I + "_window_keys");
    const auto& b = f.tensors.at("tq_" + I + "_window_values");
    if (a.shape.size() != 4 || b.shape.size() != 4 || a.shape[2] != window || b.shape[2] != window)
      throw Error("layer " + I + ": TurboQuant window length mismatch: required miss");
  }
  return offset;
}

// restoreTQLayer into a fresh layer (CacheHelpers.swift:1248-1320):
// TurboQuantKVCache(keyBits: ck bits + 1, valueBits: cv bits, sinkTokens:
// max(sinks, 4), residualTokens: max(tails, 64)), then restoreCompressed.
std::unique_ptr<Cache> load_tq_layer(const StFile& f, const std::string& I, int64_t offset,
                                     hipStream_t st) {
  std::vector<DevBuf> keep;
  auto dev = [&](const std::string& key, vkv_array* a) {
    if (!f.tensors.count(key)) {
      *a = vkv_array{};
      return;
    }
    keep.push_back(to_device(read_tensor(f, key), st, a));
  };
  auto record = [&](const std::string& pre, const std::string& meta, bool keys) {
    vkv_tq_encoded e{};
    dev(pre + "indices", &e.indices);
    if (keys) {
      dev(pre + "qjl", &e.qjl);
      dev(pre + "res_norms", &e.res_norms);
      dev(pre + "vec_norms", &e.vec_norms);
    } else {
      dev(pre + "norms", &e.vec_norms);
    }
    dev(pre + "sink", &e.sink);
    dev(pre + "tail", &e.tail);
    HostTensor sh = read_tensor(f, meta + "_shape__");
    if (sh.shape.size() != 1 || sh.shape[0] != 4) throw Error("layer " + I + ": bad TurboQuant shape");
    memcpy(e.shape, sh.data.data(), 16);
    meta_int32(f, meta + "_index_bits__", &e.index_bits);
    meta_int32(f, meta + "_seed__", &e.seed);
    return e;
  };
  vkv_tq_encoded ek = record("tq_" + I + "_ck_", "__tq_" + I + "_ck", true);
  vkv_tq_encoded ev = record("tq_" + I + "_cv_", "__tq_" + I + "_cv", false);
  vkv_array wk{}, wv{};
  dev("tq_" + I + "_window_keys", &wk);
  dev("tq_" + I + "_window_values", &wv);
  auto cnt = [](const vkv_array& a) { return a.ndim == 4 ? a.shape[2] : 0; };
  const int sink = static_cast<int>(std::max<int64_t>({cnt(ek.sink), cnt(ev.sink), 4}));
  const int res = static_cast<int>(std::max<int64_t>({cnt(ek.tail), cnt(ev.tail), 64}));
  auto c = std::make_unique<TurboQuantCache>(ek.index_bits + 1, ev.index_bits, sink, res);
  c->restore_compressed(ek, ev, offset, wk.ndim ? &wk : nullptr, wv.ndim ? &wv : nullptr, st);
  VKV_HIP(hipStreamSynchronize(st));
  if (c->offset <= 0) throw Error("layer " + I + ": the TurboQuant layer did not restore: required miss");
  return c;
}

}  // namespace

// TQDiskSerializer.serialize (version 2) for the attention layers this
// library holds: KVCacheSimple -> kind 2 (kv_i_keys / kv_i_values),
// RotatingKVCache -> kind 6 (rot_i_keys / rot_i_values + __rot_i_meta__
// [keep, maxSize, step, offset, idx]), QuantizedKVCache -> kind 5
// (qkv_i_k + __qkv_i_count__ / _offset__ / _group_size__ / _bits__), a
// compressed TurboQuantKVCache holding its encoded records -> kind 1, any
// other TurboQuantKVCache -> kind 2 from its state; an empty cache -> kind
// 4 (skip).  Scalars are 1-element int32 arrays.
int vkv_disk_cache_save(const char* path, const vkv_cache* caches, int32_t n_caches, void* stream) {
  return guarded([&] {
    if (!path) throw Error("path is NULL");
    if (n_caches < 0 || (n_caches > 0 && !caches)) throw Error("caches is NULL");
    const hipStream_t st = S(stream);
    TensorMap ts;
    ts["__jang_cache_format_version__"] = int32_vec({2});
    ts["__tq_native_marker__"] = int32_vec({1});
    for (int i = 0; i < n_caches; i++) {
      if (!caches[i]) throw Error("cache " + std::to_string(i) + " is NULL");
      Cache& c = *caches[i]->impl;
      const std::string I = std::to_string(i);
      const std::string kind_key = "__layer_kind_" + I + "__";
      const int kind = c.kind();
      if (kind == VKV_CACHE_TURBOQUANT || kind == VKV_CACHE_COMPILABLE_TURBOQUANT) {
        auto* t = static_cast<TurboQuantCache*>(&c);
        if (t->phase_ == 1 && t->ck_ && t->cv_) {
          save_tq_layer(*t, I, ts, st);
          ts[kind_key] = int32_vec({1});
          continue;
        }
      }
      auto arrays = state_to_host(c, st);
      if (kind == VKV_CACHE_QUANTIZED) {
        if (arrays.size() != 4 && arrays.size() != 6) {
          ts[kind_key] = int32_vec({4});
          continue;
        }
        const auto* q = static_cast<const QuantizedCache*>(&c);
        const int n = static_cast<int>(arrays.size());
        for (int k = 0; k < n; k++) ts["qkv_" + I + "_" + std::to_string(k)] = std::move(arrays[k]);
        ts["__qkv_" + I + "_count__"] = int32_vec({n});
        ts["__qkv_" + I + "_offset__"] = int32_vec({static_cast<int32_t>(c.current_offset())});
        ts["__qkv_" + I + "_group_size__"] = int32_vec({q->group_});
        ts["__qkv_" + I + "_bits__"] = int32_vec({q->bits_});
        ts[kind_key] = int32_vec({5});
      } else if (kind == VKV_CACHE_ROTATING || kind == VKV_CACHE_COMPILABLE_ROTATING) {
        auto info = c.meta_state();
        if (arrays.size() != 2 || info.size() != 5) {
          ts[kind_key] = int32_vec({4});
          continue;
        }
        std::vector<int32_t> m;
        for (auto& s : info) m.push_back(parse_int(s, INT32_MIN));
        if (std::find(m.begin(), m.end(), INT32_MIN) != m.end()) {
          ts[kind_key] = int32_vec({4});
          continue;
        }
        ts["rot_" + I + "_keys"] = std::move(arrays[0]);
        ts["rot_" + I + "_values"] = std::move(arrays[1]);
        ts["__rot_" + I + "_meta__"] = int32_vec(m);
        ts[kind_key] = int32_vec({6});
      } else {
        if (arrays.size() < 2) {
          ts[kind_key] = int32_vec({4});
          continue;
        }
        ts["kv_" + I + "_keys"] = std::move(arrays[0]);
        ts["kv_" + I + "_values"] = std::move(arrays[1]);
        ts[kind_key] = int32_vec({2});
      }
    }
    write_safetensors(path, ts, StrMap{{"format", "mlx"}});  // DiskCache.swift:315
  });
}

// TQDiskSerializer.deserializeV2 (:1023-1170) for kinds 1, 2, 5, 6 and 4:
// caches[i] receives the restored layer i, or NULL for a skipped layer.  A
// missing kind tag inside the layer range, an incomplete payload, a
// TurboQuant layer that does not restore or an unsupported kind (Mamba,
// composite) fails the whole record, as the reference turns them into a
// required miss.
int vkv_disk_cache_load(const char* path, void* stream, vkv_cache* caches, int32_t capacity,
                        int32_t* n_layers) {
  return guarded([&] {
    if (!path) throw Error("path is NULL");
    if (!n_layers) throw Error("n_layers is NULL");
    const hipStream_t st = S(stream);
    StFile f = read_safetensors_header(path);
    int32_t version = 0;
    if (!meta_int32(f, "__jang_cache_format_version__", &version) || version != 2)
      throw Error("not a version-2 disk cache record");
    std::map<int, int32_t> kinds;
    for (auto& kv : f.tensors) {
      const std::string& k = kv.first;
      if (k.rfind("__layer_kind_", 0) != 0 || k.size() < 16 || k.substr(k.size() - 2) != "__") continue;
      const int i = parse_int(k.substr(13, k.size() - 15), -1);
      int32_t v = 0;
      if (i >= 0 && meta_int32(f, k, &v)) kinds[i] = v;
    }
    const int n = kinds.empty() ? 0 : kinds.rbegin()->first + 1;
    *n_layers = n;
    if (!caches) return;
    if (capacity < n) throw Error("caches capacity is smaller than the record's layer count");
    for (int i = 0; i < n; i++) caches[i] = nullptr;
    // the whole record is checked before any layer is restored
    for (int i = 0; i < n; i++) {
      const std::string I = std::to_string(i);
      if (!kinds.count(i)) throw Error("layer " + I + " has no kind tag: required miss");
      const int32_t kind = kinds[i];
      auto has = [&](const std::string& k) { return f.tensors.count(k) > 0; };
      if (kind == 2 && !(has("kv_" + I + "_keys") && has("kv_" + I + "_values")))
        throw Error("layer " + I + ": incomplete kv payload");
      if (kind == 6 && !(has("rot_" + I + "_keys") && has("rot_" + I + "_values") &&
                         has("__rot_" + I + "_meta__")))
        throw Error("layer " + I + ": incomplete rotating payload");
      if (kind == 5) {
        int32_t count = 0, x = 0;
        if (!meta_int32(f, "__qkv_" + I + "_count__", &count) || (count != 4 && count != 6) ||
            !meta_int32(f, "__qkv_" + I + "_offset__", &x) ||
            !meta_int32(f, "__qkv_" + I + "_group_size__", &x) ||
            !meta_int32(f, "__qkv_" + I + "_bits__", &x))
          throw Error("layer " + I + ": incomplete quantized payload");
        for (int k = 0; k < count; k++)
          if (!has("qkv_" + I + "_" + std::to_string(k)))
            throw Error("layer " + I + ": incomplete quantized payload");
      }
      if (kind == 1) check_tq_layer(f, I);
      if (kind != 1 && kind != 2 && kind != 4 && kind != 5 && kind != 6)
        throw Error("layer " + I + ": kind " + std::to_string(kind) +
                    " (Mamba or composite) is not restored here: required miss");
    }
    std::vector<std::unique_ptr<Cache>> built(n);
    for (int i = 0; i < n; i++) {
      const std::string I = std::to_string(i);
      const int32_t kind = kinds[i];
      vkv_cache_params p{};
      if (kind == 4) continue;  // skip
      if (kind == 1) {
        built[i] = load_tq_layer(f, I, check_tq_layer(f, I), st);
      } else if (kind == 2) {
        if (!f.tensors.count("kv_" + I + "_keys") || !f.tensors.count("kv_" + I + "_values"))
          throw Error("layer " + I + ": incomplete kv payload");
        p.kind = VKV_CACHE_SIMPLE;
        auto c = make_cache(p);
        set_state_from_host(*c, {read_tensor(f, "kv_" + I + "_keys"), read_tensor(f, "kv_" + I + "_values")}, st);
        built[i] = std::move(c);
      } else if (kind == 6) {
        if (!f.tensors.count("rot_" + I + "_keys") || !f.tensors.count("rot_" + I + "_values") ||
            !f.tensors.count("__rot_" + I + "_meta__"))
          throw Error("layer " + I + ": incomplete rotating payload");
        HostTensor m = read_tensor(f, "__rot_" + I + "_meta__");
        if (m.dtype != VKV_I32 || m.shape.size() != 1 || m.shape[0] != 5)
          throw Error("layer " + I + ": bad rotating metadata");
        int32_t mv[5];
        memcpy(mv, m.data.data(), sizeof(mv));
        p.kind = VKV_CACHE_ROTATING;
        p.max_size = mv[1];
        p.keep = mv[0];
        p.step = mv[2];
        auto c = make_cache(p);
        set_state_from_host(*c, {read_tensor(f, "rot_" + I + "_keys"), read_tensor(f, "rot_" + I + "_values")}, st);
        std::vector<std::string> info;
        for (int k = 0; k < 5; k++) info.push_back(std::to_string(mv[k]));
        c->set_meta_state(info);
        built[i] = std::move(c);
      } else if (kind == 5) {
        int32_t count = 0, offset = 0, group = 0, bits = 0;
        if (!meta_int32(f, "__qkv_" + I + "_count__", &count) ||
            !meta_int32(f, "__qkv_" + I + "_offset__", &offset) ||
            !meta_int32(f, "__qkv_" + I + "_group_size__", &group) ||
            !meta_int32(f, "__qkv_" + I + "_bits__", &bits) || (count != 4 && count != 6))
          throw Error("layer " + I + ": incomplete quantized payload");
        std::vector<HostTensor> arrays;
        for (int k = 0; k < count; k++) {
          const std::string key = "qkv_" + I + "_" + std::to_string(k);
          if (!f.tensors.count(key)) throw Error("layer " + I + ": incomplete quantized payload");
          arrays.push_back(read_tensor(f, key));
        }
        p.kind = VKV_CACHE_QUANTIZED;
        p.group_size = group;
        p.bits = bits;
        auto c = make_cache(p);
        set_state_from_host(*c, arrays, st);
        c->set_meta_state({"256", std::to_string(offset), std::to_string(group), std::to_string(bits)});
        built[i] = std::move(c);
      } else {
        throw Error("layer " + I + ": kind " + std::to_string(kind) +
                    " (Mamba or composite) is not restored here: required miss");
      }
    }
    for (int i = 0; i < n; i++) {
      caches[i] = nullptr;
      if (!built[i]) continue;
      auto h = new vkv_cache_s;
      h->impl = std::move(built[i]);
      caches[i] = h;
    }
  });
}

}  // extern "C"

// ------------------------------------------- prompt caches from pool blocks

namespace {

// A one-sequence device block table for pool views (host ids uploaded).
DevBuf upload_table(const int32_t* blocks, int32_t n, const Pool& pool, hipStream_t st) {
  for (int i = 0; i < n; i++)
    if (blocks[i] < 0 || blocks[i] >= pool.p.num_blocks) throw Error("block id out of range");
  DevBuf t(static_cast<size_t>(std::max(n, 1)) * sizeof(int32_t));
  VKV_HIP(hipMemcpyAsync(t.get(), blocks, static_cast<size_t>(n) * sizeof(int32_t),
                         hipMemcpyHostToDevice, st));
  return t;
}

}  // namespace

extern "C" {

// savePromptCache's file (KVCache.swift:1620-1680) written from one
// sequence's pool blocks: per layer, an affine pool gives the six
// reference-layout QuantizedKVCache arrays (the codes as stored, no
// requantization) with metaState [256, n, group, bits]; a float pool gives
// KVCacheSimple's keys and values [1, H, n, D].
int vkv_prompt_cache_save_paged(const char* path, vkv_pool pool, const int32_t* blocks,
                                int32_t n_blocks, int64_t n_tokens, const char* const* meta_keys,
                                const char* const* meta_values, int32_t n_meta, void* stream) {
  return guarded([&] {
    if (!path) throw Error("path is NULL");
    if (!pool) throw Error("pool is NULL");
    Pool& P = *pool->impl;
    if (P.p.flags & VKV_VIEW_KEYS_ONLY) throw Error("keys-only (latent) pools have no prompt-cache form");
    if (n_tokens < 0 || n_tokens > static_cast<int64_t>(n_blocks) * P.p.block_size)
      throw Error("n_tokens does not fit the blocks");
    if (n_blocks > 0 && !blocks) throw Error("blocks is NULL");
    if (n_meta > 0 && (!meta_keys || !meta_values)) throw Error("metadata is NULL");
    const hipStream_t st = S(stream);
    DevBuf table = upload_table(blocks, n_blocks, P, st);
    const int64_t T = n_tokens, H = P.p.n_kv_heads, D = P.p.head_dim;
    const int es = elem_bytes(P.p.dtype);
    TensorMap ts;
    StrMap meta;
    for (int l = 0; l < P.p.n_layers; l++) {
      const std::string I = std::to_string(l);
      vkv_paged_view vw = P.view(l, static_cast<const int32_t*>(table.get()), std::max(n_blocks, 1),
                                 nullptr, 1, static_cast<int32_t>(T));
      KVSrc kv = kvsrc_from_view(vw);
      if (P.p.bits) {
        const int64_t W = D * P.p.bits / 32, G = D / P.p.group_size;
        for (int which = 0; which < 2; which++) {
          DevBuf c(static_cast<size_t>(std::max<int64_t>(1, H * T * W) * 4));
          DevBuf s(static_cast<size_t>(std::max<int64_t>(1, H * T * G) * es));
          DevBuf b(static_cast<size_t>(std::max<int64_t>(1, H * T * G) * es));
          if (T > 0) {
            GatherArgs g{};
            g.kv = kv;
            g.n_seqs = 1;
            g.H = static_cast<int32_t>(H);
            g.T = static_cast<int32_t>(T);
            g.D = static_cast<int32_t>(D);
            g.which = which;
            g.bits = P.p.bits;
            g.group = P.p.group_size;
            g.dtype = P.p.dtype;
            g.out = c.get();
            g.out_s = s.get();
            g.out_b = b.get();
            launch_gather(g, 1, st);
          }
          const int64_t lasts[3] = {W, G, G};
          const int dts[3] = {VKV_U32, P.p.dtype, P.p.dtype};
          DevBuf* bufs[3] = {&c, &s, &b};
          for (int i = 0; i < 3; i++) {
            vkv_array a{};
            a.data = bufs[i]->get();
            a.dtype = dts[i];
            a.ndim = 4;
            const int64_t shp[4] = {1, H, T, lasts[i]};
            int64_t stv = 1;
            for (int d = 3; d >= 0; d--) {
              a.shape[d] = shp[d];
              a.strides[d] = stv;
              stv *= shp[d];
            }
            ts[I + "." + std::to_string(3 * which + i)] = to_host(a, st);
          }
        }
        const std::string info[4] = {"256", std::to_string(T), std::to_string(P.p.group_size),
                                     std::to_string(P.p.bits)};
        for (int j = 0; j < 4; j++) meta["0." + I + "." + std::to_string(j)] = info[j];
        meta["2." + I] = "QuantizedKVCache";
      } else {
        for (int which = 0; which < 2; which++) {
          const int64_t Dw = which ? P.p.v_head_dim : D;
          DevBuf o(static_cast<size_t>(std::max<int64_t>(1, H * T * Dw) * es));
          if (T > 0) {
            GatherArgs g{};
            g.kv = kv;
            g.n_seqs = 1;
            g.H = static_cast<int32_t>(H);
            g.T = static_cast<int32_t>(T);
            g.D = static_cast<int32_t>(Dw);
            g.which = which;
            g.bits = 0;
            g.group = P.p.group_size;
            g.dtype = P.p.dtype;
            g.out = o.get();
            launch_gather(g, 0, st);
          }
          vkv_array a{};
          a.data = o.get();
          a.dtype = P.p.dtype;
          a.ndim = 4;
          const int64_t shp[4] = {1, H, T, Dw};
          int64_t stv = 1;
          for (int d = 3; d >= 0; d--) {
            a.shape[d] = shp[d];
            a.strides[d] = stv;
            stv *= shp[d];
          }
          ts[I + "." + std::to_string(which)] = to_host(a, st);
        }
        meta["0." + I + ".0"] = "";
        meta["2." + I] = "KVCache";
      }
    }
    for (int k = 0; k < n_meta; k++) {
      if (!meta_keys[k] || !meta_values[k]) throw Error("metadata entry is NULL");
      meta[std::string("1.") + meta_keys[k]] = meta_values[k];
    }
    write_safetensors(path, ts, meta);
  });
}

// loadPromptCache's file (KVCache.swift:1687-1780) read into one sequence's
// pool blocks: every layer of the pool, tokens 0 .. n-1 at block
// blocks[t / block_size], offset t % block_size.  KVCacheSimple layers are
// appended (quantized on the way for an affine pool); QuantizedKVCache
// layers whose group size and bits match an affine pool are written as
// they are (no requantization), other quantized layers are dequantized and
// appended (the reference's dequantize-store / requantize-restore,
// CacheHelpers.swift:431-552).  *n_tokens receives n.
int vkv_prompt_cache_load_paged(const char* path, vkv_pool pool, const int32_t* blocks,
                                int32_t n_blocks, int64_t* n_tokens, char* meta_buf,
                                int64_t meta_buf_len, int32_t* n_meta, void* stream) {
  return guarded([&] {
    if (!path) throw Error("path is NULL");
    if (!pool) throw Error("pool is NULL");
    Pool& P = *pool->impl;
    if (P.p.flags & VKV_VIEW_KEYS_ONLY) throw Error("keys-only (latent) pools have no prompt-cache form");
    if (n_blocks > 0 && !blocks) throw Error("blocks is NULL");
    const hipStream_t st = S(stream);
    StFile f = read_safetensors_header(path);
    const int L = P.p.n_layers;
    const int64_t H = P.p.n_kv_heads, D = P.p.head_dim;
    // validate the whole file against the pool first
    int64_t T = -1;
    std::vector<std::string> cls(L);
    std::vector<std::vector<std::string>> info(L);
    StrMap user;
    for (auto& kv : f.meta)
      if (kv.first.rfind("1.", 0) == 0) user[kv.first.substr(2)] = kv.second;
    for (int l = 0; l < L; l++) {
      const std::string I = std::to_string(l);
      auto c = f.meta.find("2." + I);
      if (c == f.meta.end()) throw Error("the file holds fewer layers than the pool");
      cls[l] = c->second;
      for (int j = 0;; j++) {
        auto m = f.meta.find("0." + I + "." + std::to_string(j));
        if (m == f.meta.end()) break;
        info[l].push_back(m->second);
      }
      const int na = cls[l] == "QuantizedKVCache" ? 6 : 2;
      if (cls[l] != "QuantizedKVCache" && cls[l] != "KVCache" && cls[l] != "KVCacheSimple")
        throw Error("layer " + I + ": class " + cls[l] + " cannot be restored into pool blocks");
      for (int j = 0; j < na; j++) {
        auto t = f.tensors.find(I + "." + std::to_string(j));
        if (t == f.tensors.end()) throw Error("layer " + I + ": missing state array " + std::to_string(j));
        const auto& sh = t->second.shape;
        if (sh.size() != 4 || sh[0] != 1 || sh[1] != H)
          throw Error("layer " + I + ": state arrays must be [1, " + std::to_string(H) + ", n, .]");
        if (T < 0) T = sh[2];
        if (sh[2] != T) throw Error("layer " + I + ": token counts differ between arrays");
        const bool codes = na == 6 && j % 3 == 0;
        if (na == 2 && (sh[3] != (j ? P.p.v_head_dim : D) || t->second.dtype != P.p.dtype))
          throw Error("layer " + I + ": keys/values do not match the pool's head dims or dtype");
        if (codes && t->second.dtype != VKV_U32) throw Error("layer " + I + ": codes must be u32");
        if (na == 6 && !codes && t->second.dtype != P.p.dtype)
          throw Error("layer " + I + ": scales/biases do not match the pool's dtype");
      }
      if (na == 6) {
        const int bits = info[l].size() >= 4 ? parse_int(info[l][3], 0) : 0;
        const int group = info[l].size() >= 3 ? parse_int(info[l][2], 0) : 0;
        if ((bits != 4 && bits != 8) || group <= 0 || D % group ||
            f.tensors[I + ".0"].shape[3] * 32 != D * bits || f.tensors[I + ".1"].shape[3] != D / group)
          throw Error("layer " + I + ": quantized arrays do not match their metaState or the head dim");
      }
    }
    if (T < 0) T = 0;
    if (T > static_cast<int64_t>(n_blocks) * P.p.block_size) throw Error("the file's tokens do not fit the blocks");
    if (n_tokens) *n_tokens = T;
    put_meta_out(user, meta_buf, meta_buf_len, n_meta);
    if (T == 0) return;
    DevBuf table = upload_table(blocks, n_blocks, P, st);
    std::vector<int32_t> slots(static_cast<size_t>(T));
    for (int64_t t = 0; t < T; t++)
      slots[t] = blocks[t / P.p.block_size] * P.p.block_size + static_cast<int32_t>(t % P.p.block_size);
    DevBuf slot_buf(slots.size() * sizeof(int32_t));
    VKV_HIP(hipMemcpyAsync(slot_buf.get(), slots.data(), slots.size() * sizeof(int32_t),
                           hipMemcpyHostToDevice, st));
    const int es = elem_bytes(P.p.dtype);
    for (int l = 0; l < L; l++) {
      const std::string I = std::to_string(l);
      // [1, H, T, D] device arrays seen as [T, H, D] rows for the append
      auto as_rows = [&](const vkv_array& a) {
        vkv_array r{};
        r.data = a.data;
        r.dtype = a.dtype;
        r.ndim = 3;
        r.shape[0] = T;
        r.shape[1] = H;
        r.shape[2] = a.shape[3];
        r.strides[0] = a.shape[3];
        r.strides[1] = T * a.shape[3];
        r.strides[2] = 1;
        return r;
      };
      if (cls[l] != "QuantizedKVCache") {
        vkv_array k, v;
        DevBuf kb = to_device(read_tensor(f, I + ".0"), st, &k);
        DevBuf vb = to_device(read_tensor(f, I + ".1"), st, &v);
        vkv_array kr = as_rows(k), vr = as_rows(v);
        P.append(l, kr, &vr, static_cast<const int32_t*>(slot_buf.get()), T, st);
        VKV_HIP(hipStreamSynchronize(st));
        continue;
      }
      const int group = parse_int(info[l][2], 64), bits = parse_int(info[l][3], 8);
      vkv_array a[6];
      std::vector<DevBuf> bufs;
      for (int j = 0; j < 6; j++) bufs.push_back(to_device(read_tensor(f, I + "." + std::to_string(j)), st, &a[j]));
      if (P.p.bits == bits && P.p.group_size == group) {
        const bool keys_only = false;
        uint8_t* base = P.mem.bytes() + static_cast<int64_t>(l) * P.layer_bytes;
        for (int which = 0; which < 2; which++) {
          ScatterCodesArgs s{};
          s.wq = static_cast<const uint32_t*>(a[3 * which].data);
          s.scales = a[3 * which + 1].data;
          s.biases = a[3 * which + 2].data;
          s.n_seqs = 1;
          s.H = static_cast<int32_t>(H);
          s.T = static_cast<int32_t>(T);
          s.D = static_cast<int32_t>(D);
          s.bits = bits;
          s.group = group;
          s.dtype = P.p.dtype;
          s.is_v = which;
          s.dst = affine_dst(base, P.block_bytes, P.head_bytes, P.p.block_size, P.L, which,
                             static_cast<int>(D / group), keys_only);
          s.dst.table = static_cast<const int32_t*>(table.get());
          s.dst.table_stride = std::max(n_blocks, 1);
          launch_scatter_codes(s, st);
        }
      } else {
        // dequantize (to the scales' dtype), then append in the pool's format
        DevBuf deq[2];
        vkv_array rows[2];
        for (int which = 0; which < 2; which++) {
          deq[which].alloc(static_cast<size_t>(std::max<int64_t>(1, H * T * D) * es));
          launch_dequantize(P.p.dtype, bits, group, static_cast<const uint32_t*>(a[3 * which].data),
                            a[3 * which + 1].data, a[3 * which + 2].data, deq[which].get(), H * T,
                            static_cast<int>(D), st);
          vkv_array d{};
          d.data = deq[which].get();
          d.dtype = P.p.dtype;
          d.ndim = 4;
          d.shape[0] = 1;
          d.shape[1] = H;
          d.shape[2] = T;
          d.shape[3] = D;
          rows[which] = as_rows(d);
        }
        P.append(l, rows[0], &rows[1], static_cast<const int32_t*>(slot_buf.get()), T, st);
      }
      VKV_HIP(hipStreamSynchronize(st));
    }
  });
}

}  // extern "C"
