// bb_gguf.hip — GGUF files on the host: the container parse (gguf.rs), the architecture check
// (config.rs:51-89), the tensor-table check (model.rs:572-584, :619-660) and the one-time load
// of a decoder into HBM (Model::load, model.rs:36-67). Host code only: the tensors go to the
// device through bb_tensor_upload, the operators and the decoder through their create calls.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <exception>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/bebelm_moe.h"
#include "bb_internal.h"

namespace {

struct Fail {
  int code;
};

[[noreturn]] void fail(int code, const std::string& msg) {
  bb::set_last_error(msg);
  throw Fail{code};
}

void need(bool ok, int code, const std::string& msg) {
  if (!ok) fail(code, msg);
}

void check_code(int rc) {
  if (rc != BB_OK) throw Fail{rc};  // the callee already set the message
}

template <class F>
int guard(F&& f) {
  try {
    bb::set_last_error("");
    f();
    return BB_OK;
  } catch (const Fail& x) {
    return x.code;
  } catch (const std::bad_alloc&) {
    bb::set_last_error("host allocation failed");
    return BB_ERR_OOM;
  } catch (const std::exception& x) {
    bb::set_last_error(x.what());
    return BB_ERR_ARG;
  } catch (...) {
    bb::set_last_error("unknown error");
    return BB_ERR_ARG;
  }
}

// Metadata value types, the on-disk discriminants (gguf.rs:61-75).
enum Vt : uint32_t {
  VT_U8 = 0, VT_I8 = 1, VT_U16 = 2, VT_I16 = 3, VT_U32 = 4, VT_I32 = 5, VT_F32 = 6,
  VT_BOOL = 7, VT_STRING = 8, VT_ARRAY = 9, VT_U64 = 10, VT_I64 = 11, VT_F64 = 12, VT_COUNT = 13
};

struct Value {
  uint32_t type = 0;
  uint64_t bits = 0;           // scalar payload as read (zero-extended raw little-endian bits)
  std::string str;             // VT_STRING
  uint32_t elem_type = 0;      // VT_ARRAY
  std::vector<Value> items;    // VT_ARRAY
};

bool is_int(uint32_t t) {
  return t == VT_U8 || t == VT_I8 || t == VT_U16 || t == VT_I16 || t == VT_U32 || t == VT_I32 || t == VT_U64 ||
         t == VT_I64;
}

// `v as u32` for each integer variant (gguf.rs:200-212): signed values sign-extend first.
uint32_t as_u32(const Value& v) {
  switch (v.type) {
    case VT_I8: return (uint32_t)(int32_t)(int8_t)(uint8_t)v.bits;
    case VT_I16: return (uint32_t)(int32_t)(int16_t)(uint16_t)v.bits;
    default: return (uint32_t)v.bits;  // u8/u16/u32 widen, i32 reinterprets, u64/i64 truncate
  }
}

// (elements, bytes) per block of each ggml type the reference models (tensor.rs:41-93).
bool ggml_block(uint32_t t, uint64_t& elems, uint64_t& bytes) {
  switch (t) {
    case 0: elems = 1; bytes = 4; return true;      // F32
    case 1: elems = 1; bytes = 2; return true;      // F16
    case 2: elems = 32; bytes = 18; return true;    // Q4_0
    case 3: elems = 32; bytes = 20; return true;    // Q4_1
    case 6: elems = 32; bytes = 22; return true;    // Q5_0
    case 7: elems = 32; bytes = 24; return true;    // Q5_1
    case 8: elems = 32; bytes = 34; return true;    // Q8_0
    case 9: elems = 32; bytes = 36; return true;    // Q8_1
    case 10: elems = 256; bytes = 84; return true;  // Q2_K
    case 11: elems = 256; bytes = 110; return true; // Q3_K
    case 12: elems = 256; bytes = 144; return true; // Q4_K
    case 13: elems = 256; bytes = 176; return true; // Q5_K
    case 14: elems = 256; bytes = 210; return true; // Q6_K
    case 15: elems = 256; bytes = 292; return true; // Q8_K
    case 24: elems = 1; bytes = 1; return true;     // I8
    case 25: elems = 1; bytes = 2; return true;     // I16
    case 26: elems = 1; bytes = 4; return true;     // I32
    case 27: elems = 1; bytes = 8; return true;     // I64
    case 28: elems = 1; bytes = 8; return true;     // F64
    case 30: elems = 1; bytes = 2; return true;     // BF16
    default: return false;
  }
}

// Strict UTF-8 (what String::from_utf8 accepts): no overlong forms, no surrogates, <= U+10FFFF.
bool valid_utf8(const uint8_t* p, size_t n) {
  size_t i = 0;
  while (i < n) {
    const uint8_t c = p[i];
    if (c < 0x80) {
      ++i;
      continue;
    }
    size_t len;
    uint8_t lo = 0x80, hi = 0xBF;
    if (c >= 0xC2 && c <= 0xDF) {
      len = 2;
    } else if (c >= 0xE0 && c <= 0xEF) {
      len = 3;
      if (c == 0xE0) lo = 0xA0;
      if (c == 0xED) hi = 0x9F;
    } else if (c >= 0xF0 && c <= 0xF4) {
      len = 4;
      if (c == 0xF0) lo = 0x90;
      if (c == 0xF4) hi = 0x8F;
    } else {
      return false;
    }
    if (n - i < len) return false;
    if (p[i + 1] < lo || p[i + 1] > hi) return false;
    for (size_t k = 2; k < len; ++k)
      if (p[i + k] < 0x80 || p[i + k] > 0xBF) return false;
    i += len;
  }
  return true;
}

// A little-endian, bounds-checked cursor (gguf.rs:377-429).
struct Reader {
  const uint8_t* buf;
  size_t len, pos = 0;

  const uint8_t* take(size_t n) {
    size_t end;
    if (__builtin_add_overflow(pos, n, &end) || end > len)
      fail(BB_ERR_FORMAT, "unexpected end of file: need " + std::to_string(n) + " bytes at offset " +
                              std::to_string(pos) + ", file is " + std::to_string(len) + " bytes");
    const uint8_t* s = buf + pos;
    pos = end;
    return s;
  }
  uint64_t le(size_t n) {
    const uint8_t* s = take(n);
    uint64_t v = 0;
    for (size_t i = 0; i < n; ++i) v |= (uint64_t)s[i] << (8 * i);
    return v;
  }
  uint32_t u32() { return (uint32_t)le(4); }
  uint64_t u64() { return le(8); }
  std::string str() {
    const uint64_t n = u64();
    const uint8_t* s = take((size_t)n);
    if (!valid_utf8(s, (size_t)n)) fail(BB_ERR_FORMAT, "invalid UTF-8 in a GGUF string");
    return std::string(reinterpret_cast<const char*>(s), (size_t)n);
  }
};

uint32_t value_type(uint32_t v) {
  if (v >= VT_COUNT) fail(BB_ERR_FORMAT, "unknown metadata value type " + std::to_string(v));
  return v;
}

// read_value (gguf.rs:343-369). Nested arrays recurse as in the reference; the depth is capped
// so a crafted file cannot exhaust the stack.
Value read_value(Reader& r, uint32_t vt, int depth) {
  Value v;
  v.type = vt;
  switch (vt) {
    case VT_U8: case VT_I8: case VT_BOOL: v.bits = r.le(1); break;
    case VT_U16: case VT_I16: v.bits = r.le(2); break;
    case VT_U32: case VT_I32: case VT_F32: v.bits = r.le(4); break;
    case VT_U64: case VT_I64: case VT_F64: v.bits = r.le(8); break;
    case VT_STRING: v.str = r.str(); break;
    case VT_ARRAY: {
      if (depth > 64) fail(BB_ERR_FORMAT, "metadata arrays nested deeper than 64 levels");
      v.elem_type = r.u32();
      const uint32_t et = value_type(v.elem_type);
      const uint64_t n = r.u64();
      v.items.reserve((size_t)std::min<uint64_t>(n, 4096));  // the length is not trusted
      for (uint64_t i = 0; i < n; ++i) v.items.push_back(read_value(r, et, depth + 1));
      break;
    }
  }
  return v;
}

struct Tensor {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t type;
  uint64_t offset, data_start, data_len;
};

}  // namespace

struct bb_gguf {
  // Backing bytes: a read-only mapping of the file, or an owned copy (bb_gguf_open_bytes).
  const uint8_t* data = nullptr;
  size_t len = 0;
  void* map = nullptr;
  std::vector<uint8_t> owned;
  uint32_t version = 0;
  uint64_t alignment = 32;  // gguf.rs:18
  uint64_t data_offset = 0;
  std::vector<std::pair<std::string, Value>> meta;
  std::unordered_map<std::string, size_t> meta_index;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> tensor_index;

  ~bb_gguf() {
    if (map) munmap(map, len);
  }
  const Value* get(const char* key) const {
    if (!key) return nullptr;
    auto it = meta_index.find(key);
    return it == meta_index.end() ? nullptr : &meta[it->second].second;
  }
};

namespace {

// parse (gguf.rs:280-341).
void parse(bb_gguf& g) {
  Reader r{g.data, g.len};
  const uint8_t* m = r.take(4);
  if (std::memcmp(m, "GGUF", 4) != 0)
    fail(BB_ERR_FORMAT, "not a GGUF file (magic = [" + std::to_string(m[0]) + ", " + std::to_string(m[1]) + ", " +
                            std::to_string(m[2]) + ", " + std::to_string(m[3]) + "])");
  g.version = r.u32();
  if (g.version != 2 && g.version != 3) fail(BB_ERR_FORMAT, "unsupported GGUF version " + std::to_string(g.version));
  const uint64_t tensor_count = r.u64();
  const uint64_t kv_count = r.u64();

  for (uint64_t i = 0; i < kv_count; ++i) {
    std::string key = r.str();
    const uint32_t vt = value_type(r.u32());
    Value v = read_value(r, vt, 0);
    auto it = g.meta_index.find(key);
    if (it != g.meta_index.end()) {
      g.meta[it->second].second = std::move(v);  // HashMap::insert keeps the last value
    } else {
      g.meta_index.emplace(key, g.meta.size());
      g.meta.emplace_back(std::move(key), std::move(v));
    }
  }

  g.alignment = 32;
  if (const Value* a = g.get("general.alignment")) {
    if (a->type == VT_U32 || a->type == VT_U64) g.alignment = a->bits;
  }

  struct Raw {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type;
    uint64_t offset;
  };
  std::vector<Raw> raw;
  raw.reserve((size_t)std::min<uint64_t>(tensor_count, 4096));
  for (uint64_t i = 0; i < tensor_count; ++i) {
    Raw t;
    t.name = r.str();
    const uint32_t nd = r.u32();
    for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(r.u64());
    t.type = r.u32();
    t.offset = r.u64();
    raw.push_back(std::move(t));
  }

  // The tensor-data section starts at the next `alignment` boundary (gguf.rs:319, :371-375).
  const uint64_t pos = r.pos;
  g.data_offset = g.alignment == 0 ? pos : (pos / g.alignment + (pos % g.alignment != 0)) * g.alignment;

  for (auto& t : raw) {
    uint64_t be, bb_;
    bool ok = ggml_block(t.type, be, bb_);
    uint64_t n = 1;
    bool overflow = false;
    for (uint64_t d : t.dims) overflow |= __builtin_mul_overflow(n, d, &n);
    if (!ok || n % be != 0)
      fail(BB_ERR_FORMAT, "tensor '" + t.name + "' has unmodeled ggml type " + std::to_string(t.type));
    // An element count or range that does not fit 64 bits cannot lie inside the file.
    uint64_t data_len = 0, start = 0, end = 0;
    overflow |= __builtin_mul_overflow(n / be, bb_, &data_len);
    overflow |= __builtin_add_overflow(g.data_offset, t.offset, &start);
    overflow |= __builtin_add_overflow(start, data_len, &end);
    if (overflow || end > (uint64_t)g.len)
      fail(BB_ERR_FORMAT, "tensor '" + t.name + "' data range falls outside the file");
    g.tensors.push_back(Tensor{std::move(t.name), std::move(t.dims), t.type, t.offset, start, data_len});
  }
  // Model::load's by_name map (model.rs:40-45) is collected in table order, so a repeated name
  // resolves to its last entry.
  for (size_t i = 0; i < g.tensors.size(); ++i) g.tensor_index[g.tensors[i].name] = i;
}

const bb_gguf& need_g(const bb_gguf* g) {
  need(g != nullptr, BB_ERR_ARG, "null GGUF handle");
  return *g;
}

const Value& need_key(const bb_gguf& g, const char* key) {
  need(key != nullptr, BB_ERR_ARG, "null key");
  const Value* v = g.get(key);
  if (!v) fail(BB_ERR_MISSING, std::string("missing metadata ") + key);
  return *v;
}

// f32 as Rust's Display prints it: the shortest decimal that reads back to the same value, in
// positional notation.
std::string rust_f32(float v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
  char buf[64];
  int prec = 0;
  for (; prec < 9; ++prec) {
    std::snprintf(buf, sizeof buf, "%.*e", prec, (double)v);
    if (std::strtof(buf, nullptr) == v) break;
  }
  // buf = [-]d.ddde[+-]XX -> digits and exponent
  std::string s(buf);
  bool neg = s[0] == '-';
  if (neg) s = s.substr(1);
  const size_t e = s.find('e');
  int exp10 = std::atoi(s.c_str() + e + 1);
  std::string digits;
  for (size_t i = 0; i < e; ++i)
    if (s[i] != '.') digits += s[i];
  std::string out;
  const int point = exp10 + 1;  // digits before the decimal point
  if (point <= 0) {
    out = "0." + std::string((size_t)-point, '0') + digits;
  } else if ((size_t)point >= digits.size()) {
    out = digits + std::string((size_t)point - digits.size(), '0');
  } else {
    out = digits.substr(0, (size_t)point) + "." + digits.substr((size_t)point);
  }
  if (out.find('.') != std::string::npos) {
    while (out.back() == '0') out.pop_back();
    if (out.back() == '.') out.pop_back();
  }
  return (neg && out != "0" ? "-" : "") + out;
}

std::string rust_dims(const std::vector<uint64_t>& d) {
  std::string s = "[";
  for (size_t i = 0; i < d.size(); ++i) s += (i ? ", " : "") + std::to_string(d[i]);
  return s + "]";
}

// The sizes Model reads, from the file's lfm2moe.* keys (the keys config::validate checks).
struct Arch {
  std::string prefix;
  uint32_t n_layers, hidden, vocab, n_heads, n_experts, n_used, dense_ff, moe_ff, n_dense, l_cache;
  float freq_base, eps;
  std::vector<uint32_t> kv_heads;  // per layer; 0 on conv layers
  uint32_t head_dim;
  bool attention(size_t i) const { return kv_heads[i] != 0; }
  bool dense(size_t i) const { return i < n_dense; }
};

uint32_t meta_u32(const bb_gguf& g, const std::string& key) {
  const Value& v = need_key(g, key.c_str());
  if (!is_int(v.type)) fail(BB_ERR_MISSING, "missing metadata " + key);
  return as_u32(v);
}

float meta_f32(const bb_gguf& g, const std::string& key) {
  const Value& v = need_key(g, key.c_str());
  if (v.type == VT_F32) {
    float f;
    uint32_t b = (uint32_t)v.bits;
    std::memcpy(&f, &b, 4);
    return f;
  }
  if (v.type == VT_F64) {
    double d;
    std::memcpy(&d, &v.bits, 8);
    return (float)d;
  }
  fail(BB_ERR_MISSING, "missing metadata " + key);
}

const std::string& meta_str(const bb_gguf& g, const char* key, const char* missing) {
  const Value* v = g.get(key);
  if (!v || v->type != VT_STRING) fail(BB_ERR_MISSING, missing);
  return v->str;
}

bool u32_array(const Value& v, std::vector<uint32_t>& out) {
  if (v.type != VT_ARRAY) return false;
  out.clear();
  for (const Value& it : v.items) {
    if (!is_int(it.type)) return false;
    out.push_back(as_u32(it));
  }
  return true;
}

Arch read_arch(const bb_gguf& g) {
  Arch a;
  a.prefix = meta_str(g, "general.architecture", "missing general.architecture") + ".";
  const std::string& p = a.prefix;
  a.n_layers = meta_u32(g, p + "block_count");
  a.hidden = meta_u32(g, p + "embedding_length");
  a.vocab = meta_u32(g, p + "vocab_size");
  a.n_heads = meta_u32(g, p + "attention.head_count");
  a.n_experts = meta_u32(g, p + "expert_count");
  a.n_used = meta_u32(g, p + "expert_used_count");
  a.dense_ff = meta_u32(g, p + "feed_forward_length");
  a.moe_ff = meta_u32(g, p + "expert_feed_forward_length");
  a.n_dense = meta_u32(g, p + "leading_dense_block_count");
  a.l_cache = meta_u32(g, p + "shortconv.l_cache");
  a.freq_base = meta_f32(g, p + "rope.freq_base");
  a.eps = meta_f32(g, p + "attention.layer_norm_rms_epsilon");
  const std::string kvk = p + "attention.head_count_kv";
  const Value* kv = g.get(kvk.c_str());
  if (!kv || !u32_array(*kv, a.kv_heads)) fail(BB_ERR_MISSING, "attention.head_count_kv missing or not an array");
  need(a.kv_heads.size() == a.n_layers, BB_ERR_FORMAT,
       "head_count_kv has " + std::to_string(a.kv_heads.size()) + " entries, expected " + std::to_string(a.n_layers));
  need(a.n_layers >= 1 && a.hidden >= 1 && a.n_heads >= 1 && a.hidden % a.n_heads == 0, BB_ERR_FORMAT,
       "embedding_length must be a positive multiple of attention.head_count");
  a.head_dim = a.hidden / a.n_heads;
  return a;
}

// expected_tensors (model.rs:619-660) for the file's sizes: GGUF dims [in, out] of y = W·x.
std::vector<std::pair<std::string, std::vector<uint64_t>>> expected_tensors(const Arch& a) {
  const uint64_t h = a.hidden;
  std::vector<std::pair<std::string, std::vector<uint64_t>>> v = {
      {"token_embd.weight", {h, a.vocab}},
      {"token_embd_norm.weight", {h}},
  };
  for (uint32_t i = 0; i < a.n_layers; ++i) {
    const std::string p = "blk." + std::to_string(i) + ".";
    v.push_back({p + "attn_norm.weight", {h}});
    v.push_back({p + "ffn_norm.weight", {h}});
    if (a.attention(i)) {
      const uint64_t kv = (uint64_t)a.kv_heads[i] * a.head_dim;
      v.push_back({p + "attn_q.weight", {h, h}});
      v.push_back({p + "attn_k.weight", {h, kv}});
      v.push_back({p + "attn_v.weight", {h, kv}});
      v.push_back({p + "attn_output.weight", {h, h}});
      v.push_back({p + "attn_q_norm.weight", {a.head_dim}});
      v.push_back({p + "attn_k_norm.weight", {a.head_dim}});
    } else {
      v.push_back({p + "shortconv.in_proj.weight", {h, 3 * h}});
      v.push_back({p + "shortconv.conv.weight", {a.l_cache, h}});
      v.push_back({p + "shortconv.out_proj.weight", {h, h}});
    }
    if (a.dense(i)) {
      v.push_back({p + "ffn_gate.weight", {h, a.dense_ff}});
      v.push_back({p + "ffn_up.weight", {h, a.dense_ff}});
      v.push_back({p + "ffn_down.weight", {a.dense_ff, h}});
    } else {
      v.push_back({p + "ffn_gate_inp.weight", {h, a.n_experts}});
      v.push_back({p + "exp_probs_b.bias", {a.n_experts}});
      v.push_back({p + "ffn_gate_exps.weight", {h, a.moe_ff, a.n_experts}});
      v.push_back({p + "ffn_up_exps.weight", {h, a.moe_ff, a.n_experts}});
      v.push_back({p + "ffn_down_exps.weight", {a.moe_ff, h, a.n_experts}});
    }
  }
  return v;
}

size_t find_tensor(const bb_gguf& g, const std::string& name) {
  auto it = g.tensor_index.find(name);
  if (it == g.tensor_index.end()) fail(BB_ERR_MISSING, "missing tensor " + name);
  return it->second;
}

// check_tensors (model.rs:572-584).
size_t check_tensors(const bb_gguf& g, const Arch& a) {
  const auto list = expected_tensors(a);
  for (const auto& [name, shape] : list) {
    const Tensor& t = g.tensors[find_tensor(g, name)];
    if (t.dims != shape)
      fail(BB_ERR_FORMAT, "tensor " + name + ": shape " + rust_dims(t.dims) + " != expected " + rust_dims(shape));
  }
  return list.size();
}

// LFM2.5-8B-A1B's constants (config.rs:12-38).
constexpr uint32_t C_N_LAYERS = 24, C_HIDDEN = 2048, C_VOCAB = 128000, C_N_HEADS = 32, C_N_KV_HEADS = 8,
                   C_DENSE_FF = 7168, C_MOE_FF = 1792, C_N_EXPERTS = 32, C_N_USED = 4, C_N_DENSE = 2, C_L_CACHE = 3;
constexpr float C_ROPE_THETA = 5000000.0f, C_RMS_EPS = 1e-5f;
constexpr uint32_t C_ATTENTION_LAYERS[6] = {2, 6, 10, 14, 18, 21};

void expect_u32(const bb_gguf& g, const char* key, uint32_t want) {
  const Value* v = g.get(key);
  if (!v || !is_int(v->type)) fail(BB_ERR_MISSING, std::string("missing metadata ") + key);
  const uint32_t got = as_u32(*v);
  if (got != want)
    fail(BB_ERR_FORMAT, std::string(key) + ": expected " + std::to_string(want) + ", got " + std::to_string(got));
}

void expect_f32(const bb_gguf& g, const char* key, float want, float tol) {
  const float got = meta_f32(g, key);
  if (std::fabs(got - want) > tol)  // f32 arithmetic, as config.rs:101; a NaN passes there too
    fail(BB_ERR_FORMAT, std::string(key) + ": expected " + rust_f32(want) + ", got " + rust_f32(got));
}

// Rust's `{:?}` of a str: quoted, with the escapes str::escape_debug applies to ASCII.
std::string rust_debug_str(const std::string& s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      case '\0': o += "\\0"; break;
      default:
        if (c < 0x20 || c == 0x7f) {
          char b[12];
          std::snprintf(b, sizeof b, "\\u{%x}", c);
          o += b;
        } else {
          o += (char)c;
        }
    }
  }
  return o + "\"";
}

// config::validate (config.rs:51-89), checks and messages in its order.
void validate(const bb_gguf& g) {
  const std::string& arch = meta_str(g, "general.architecture", "missing general.architecture");
  if (arch != "lfm2moe")
    fail(BB_ERR_FORMAT, "architecture: expected \"lfm2moe\", got " + rust_debug_str(arch));
  expect_u32(g, "lfm2moe.block_count", C_N_LAYERS);
  expect_u32(g, "lfm2moe.embedding_length", C_HIDDEN);
  expect_u32(g, "lfm2moe.vocab_size", C_VOCAB);
  expect_u32(g, "lfm2moe.attention.head_count", C_N_HEADS);
  expect_u32(g, "lfm2moe.expert_count", C_N_EXPERTS);
  expect_u32(g, "lfm2moe.expert_used_count", C_N_USED);
  expect_u32(g, "lfm2moe.feed_forward_length", C_DENSE_FF);
  expect_u32(g, "lfm2moe.expert_feed_forward_length", C_MOE_FF);
  expect_u32(g, "lfm2moe.leading_dense_block_count", C_N_DENSE);
  expect_u32(g, "lfm2moe.shortconv.l_cache", C_L_CACHE);
  expect_f32(g, "lfm2moe.rope.freq_base", C_ROPE_THETA, 1.0f);
  expect_f32(g, "lfm2moe.attention.layer_norm_rms_epsilon", C_RMS_EPS, 1e-9f);
  std::vector<uint32_t> kv;
  const Value* v = g.get("lfm2moe.attention.head_count_kv");
  if (!v || !u32_array(*v, kv)) fail(BB_ERR_MISSING, "attention.head_count_kv missing or not an array");
  if (kv.size() != C_N_LAYERS)
    fail(BB_ERR_FORMAT,
         "head_count_kv has " + std::to_string(kv.size()) + " entries, expected " + std::to_string(C_N_LAYERS));
  for (size_t i = 0; i < kv.size(); ++i) {
    bool att = false;
    for (uint32_t l : C_ATTENTION_LAYERS) att |= (l == i);
    const uint32_t want = att ? C_N_KV_HEADS : 0;
    if (kv[i] != want)
      fail(BB_ERR_FORMAT, "layer " + std::to_string(i) + ": head_count_kv=" + std::to_string(kv[i]) + ", expected " +
                              std::to_string(want) + " (schedule mismatch)");
  }
}

bb_gguf* open_backing(bb_gguf* g) {
  try {
    parse(*g);
  } catch (...) {
    delete g;
    throw;
  }
  return g;
}

}  // namespace

int bb_gguf_open(const char* path, bb_gguf** out) {
  return guard([&] {
    need(path != nullptr && out != nullptr, BB_ERR_ARG, "null argument");
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    auto io_fail = [&](int err) {
      fail(BB_ERR_IO, std::string("io error: ") + std::strerror(err) + " (os error " + std::to_string(err) + ")");
    };
    if (fd < 0) io_fail(errno);
    struct stat st;
    if (fstat(fd, &st) != 0) {
      const int e = errno;
      ::close(fd);
      io_fail(e);
    }
    auto* g = new bb_gguf();
    g->len = (size_t)st.st_size;
    if (g->len > 0) {
      void* p = mmap(nullptr, g->len, PROT_READ, MAP_PRIVATE, fd, 0);
      if (p == MAP_FAILED) {
        const int e = errno;
        ::close(fd);
        delete g;
        io_fail(e);
      }
      g->map = p;
      g->data = static_cast<const uint8_t*>(p);
    }
    ::close(fd);  // the mapping stays valid
    *out = open_backing(g);
  });
}

int bb_gguf_open_bytes(const void* bytes, size_t n, bb_gguf** out) {
  return guard([&] {
    need(out != nullptr && (bytes != nullptr || n == 0), BB_ERR_ARG, "null argument");
    auto* g = new bb_gguf();
    g->owned.assign(static_cast<const uint8_t*>(bytes), static_cast<const uint8_t*>(bytes) + n);
    g->data = g->owned.data();
    g->len = n;
    *out = open_backing(g);
  });
}

int bb_gguf_close(bb_gguf* g) {
  return guard([&] { delete g; });
}

int bb_gguf_header(const bb_gguf* gp, uint32_t* version, uint64_t* alignment, uint64_t* data_offset,
                   size_t* n_tensors, size_t* n_metadata) {
  return guard([&] {
    const bb_gguf& g = need_g(gp);
    if (version) *version = g.version;
    if (alignment) *alignment = g.alignment;
    if (data_offset) *data_offset = g.data_offset;
    if (n_tensors) *n_tensors = g.tensors.size();
    if (n_metadata) *n_metadata = g.meta.size();
  });
}

int bb_gguf_tensor(const bb_gguf* gp, size_t index, bb_gguf_tensor_info* info) {
  return guard([&] {
    const bb_gguf& g = need_g(gp);
    need(info != nullptr, BB_ERR_ARG, "null argument");
    need(index < g.tensors.size(), BB_ERR_ARG, "tensor index out of range");
    const Tensor& t = g.tensors[index];
    info->name = t.name.c_str();
    info->n_dims = (uint32_t)t.dims.size();
    info->dims = t.dims.data();
    info->ggml_type = t.type;
    info->offset = t.offset;
    info->data_start = t.data_start;
    info->data_len = t.data_len;
  });
}

int bb_gguf_find_tensor(const bb_gguf* gp, const char* name, size_t* index) {
  return guard([&] {
    const bb_gguf& g = need_g(gp);
    need(name != nullptr && index != nullptr, BB_ERR_ARG, "null argument");
    *index = find_tensor(g, name);
  });
}

int bb_gguf_tensor_data(const bb_gguf* gp, size_t index, const void** data, size_t* nbytes) {
  return guard([&] {
    const bb_gguf& g = need_g(gp);
    need(data != nullptr && nbytes != nullptr, BB_ERR_ARG, "null argument");
    need(index < g.tensors.size(), BB_ERR_ARG, "tensor index out of range");
    const Tensor& t = g.tensors[index];
    *data = g.data + t.data_start;
    *nbytes = (size_t)t.data_len;
  });
}

int bb_gguf_meta_key(const bb_gguf* gp, size_t index, const char** key) {
  return guard([&] {
    const bb_gguf& g = need_g(gp);
    need(key != nullptr, BB_ERR_ARG, "null argument");
    need(index < g.meta.size(), BB_ERR_ARG, "metadata index out of range");
    *key = g.meta[index].first.c_str();
  });
}

int bb_gguf_meta_type(const bb_gguf* gp, const char* key, uint32_t* value_type, uint32_t* elem_type, size_t* n_items) {
  return guard([&] {
    const Value& v = need_key(need_g(gp), key);
    if (value_type) *value_type = v.type;
    if (elem_type) *elem_type = v.type == VT_ARRAY ? v.elem_type : 0;
    if (n_items) *n_items = v.type == VT_ARRAY ? v.items.size() : 0;
  });
}

int bb_gguf_get_u32(const bb_gguf* gp, const char* key, uint32_t* value) {
  return guard([&] {
    need(value != nullptr, BB_ERR_ARG, "null argument");
    const Value& v = need_key(need_g(gp), key);
    if (!is_int(v.type)) fail(BB_ERR_MISSING, std::string("metadata ") + key + " is not an integer");
    *value = as_u32(v);
  });
}

int bb_gguf_get_f32(const bb_gguf* gp, const char* key, float* value) {
  return guard([&] {
    need(value != nullptr, BB_ERR_ARG, "null argument");
    need(key != nullptr, BB_ERR_ARG, "null key");
    *value = meta_f32(need_g(gp), key);
  });
}

int bb_gguf_get_str(const bb_gguf* gp, const char* key, const char** str, size_t* len) {
  return guard([&] {
    need(str != nullptr && len != nullptr, BB_ERR_ARG, "null argument");
    const Value& v = need_key(need_g(gp), key);
    if (v.type != VT_STRING) fail(BB_ERR_MISSING, std::string("metadata ") + key + " is not a string");
    *str = v.str.data();
    *len = v.str.size();
  });
}

int bb_gguf_get_u32_array(const bb_gguf* gp, const char* key, uint32_t* out, size_t cap, size_t* n_items) {
  return guard([&] {
    need(n_items != nullptr && (out != nullptr || cap == 0), BB_ERR_ARG, "null argument");
    const Value& v = need_key(need_g(gp), key);
    std::vector<uint32_t> vals;
    if (!u32_array(v, vals)) fail(BB_ERR_MISSING, std::string("metadata ") + key + " is not an integer array");
    *n_items = vals.size();
    for (size_t i = 0; i < vals.size() && i < cap; ++i) out[i] = vals[i];
  });
}

int bb_gguf_get_str_item(const bb_gguf* gp, const char* key, size_t index, const char** str, size_t* len) {
  return guard([&] {
    need(str != nullptr && len != nullptr, BB_ERR_ARG, "null argument");
    const Value& v = need_key(need_g(gp), key);
    bool all_str = v.type == VT_ARRAY;
    if (all_str)
      for (const Value& it : v.items) all_str &= it.type == VT_STRING;
    if (!all_str) fail(BB_ERR_MISSING, std::string("metadata ") + key + " is not a string array");
    need(index < v.items.size(), BB_ERR_ARG, "array index out of range");
    *str = v.items[index].str.data();
    *len = v.items[index].str.size();
  });
}

int bb_gguf_validate(const bb_gguf* gp) {
  return guard([&] { validate(need_g(gp)); });
}

int bb_gguf_check_tensors(const bb_gguf* gp, size_t* n_expected) {
  return guard([&] {
    const bb_gguf& g = need_g(gp);
    const size_t n = check_tensors(g, read_arch(g));
    if (n_expected) *n_expected = n;
  });
}

int bb_gguf_upload(bb_ctx* ctx, const bb_gguf* gp, size_t index, bb_tensor** out) {
  return guard([&] {
    const bb_gguf& g = need_g(gp);
    need(index < g.tensors.size(), BB_ERR_ARG, "tensor index out of range");
    const Tensor& t = g.tensors[index];
    need(t.dims.size() >= 1 && t.dims.size() <= 4, BB_ERR_SHAPE, "tensor " + t.name + " has more than 4 dims");
    check_code(bb_tensor_upload(ctx, t.type, g.data + t.data_start, (size_t)t.data_len, t.dims.data(),
                                (int)t.dims.size(), out));
  });
}

int bb_model_load(bb_ctx* ctx, const bb_gguf* gp, bb_model** out) {
  return guard([&] {
    const bb_gguf& g = need_g(gp);
    need(ctx != nullptr && out != nullptr, BB_ERR_ARG, "null argument");
    const Arch a = read_arch(g);
    check_tensors(g, a);

    bb::ModelOwned own;
    std::vector<bb_tensor*> transient;  // MoE uploads, freed once bb_moe_create has packed them
    auto cleanup = [&] {
      for (bb_tensor* t : transient) (void)bb_tensor_free(t);
      transient.clear();
    };
    // precompute_f32 (model.rs:54-67): the small tensors the forward pass reads as f32 slices.
    std::vector<std::vector<float>> host_f32;
    auto f32_of = [&](const std::string& name) -> const float* {
      const Tensor& t = g.tensors[find_tensor(g, name)];
      need(t.type == BB_F32, BB_ERR_DTYPE, "f32 tensor not precomputed: " + name);
      host_f32.emplace_back(t.data_len / 4);
      std::memcpy(host_f32.back().data(), g.data + t.data_start, t.data_len);
      return host_f32.back().data();
    };
    auto upload = [&](const std::string& name, std::vector<bb_tensor*>& into) -> bb_tensor* {
      bb_tensor* t = nullptr;
      check_code(bb_gguf_upload(ctx, &g, find_tensor(g, name), &t));
      into.push_back(t);
      return t;
    };
    try {
      std::vector<bb_decoder_layer> layers(a.n_layers);
      for (uint32_t i = 0; i < a.n_layers; ++i) {
        const std::string p = "blk." + std::to_string(i) + ".";
        bb_decoder_layer& D = layers[i];
        D = bb_decoder_layer{};
        D.attn_norm = f32_of(p + "attn_norm.weight");
        D.ffn_norm = f32_of(p + "ffn_norm.weight");
        if (a.attention(i)) {
          bb_tensor* q = upload(p + "attn_q.weight", own.tensors);
          bb_tensor* k = upload(p + "attn_k.weight", own.tensors);
          bb_tensor* v = upload(p + "attn_v.weight", own.tensors);
          bb_tensor* o = upload(p + "attn_output.weight", own.tensors);
          const float* qn = f32_of(p + "attn_q_norm.weight");
          const float* kn = f32_of(p + "attn_k_norm.weight");
          check_code(bb_attn_op_create(ctx, q, k, v, o, qn, kn, a.n_heads, a.kv_heads[i], a.eps, a.freq_base, &D.attn));
          own.attn.push_back(D.attn);
        } else {
          bb_tensor* in = upload(p + "shortconv.in_proj.weight", own.tensors);
          const float* cw = f32_of(p + "shortconv.conv.weight");
          bb_tensor* o = upload(p + "shortconv.out_proj.weight", own.tensors);
          check_code(bb_conv_op_create(ctx, in, cw, a.l_cache, o, &D.conv));
          own.conv.push_back(D.conv);
        }
        if (a.dense(i)) {
          bb_tensor* gt = upload(p + "ffn_gate.weight", own.tensors);
          bb_tensor* up = upload(p + "ffn_up.weight", own.tensors);
          bb_tensor* dn = upload(p + "ffn_down.weight", own.tensors);
          check_code(bb_dense_create(ctx, gt, up, dn, &D.dense));
          own.dense.push_back(D.dense);
        } else {
          bb_tensor* r = upload(p + "ffn_gate_inp.weight", transient);
          const float* bias = f32_of(p + "exp_probs_b.bias");
          bb_tensor* gt = upload(p + "ffn_gate_exps.weight", transient);
          bb_tensor* up = upload(p + "ffn_up_exps.weight", transient);
          bb_tensor* dn = upload(p + "ffn_down_exps.weight", transient);
          check_code(bb_moe_create(ctx, r, bias, gt, up, dn, (int)a.n_used, &D.moe));
          own.moe.push_back(D.moe);
          cleanup();
        }
      }
      bb_tensor* te = upload("token_embd.weight", own.tensors);
      const float* fin = f32_of("token_embd_norm.weight");
      bb_model* m = nullptr;
      check_code(bb_model_create(ctx, te, fin, layers.data(), layers.size(), a.eps, &m));
      bb::model_adopt(m, std::move(own));
      *out = m;
    } catch (...) {
      cleanup();
      bb::free_owned(own);
      throw;
    }
  });
}
