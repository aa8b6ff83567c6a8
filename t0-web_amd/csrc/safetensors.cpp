// The real-checkpoint entry: an F32 `model.safetensors` plus its `config.json`
// exported to GGUF with the reference's policy, or loaded straight onto the
// device through that export.
//
// Reference: Weights::load_bytes (crates/t0-core/src/weights.rs:115-140, via
// the `safetensors` crate, 0.4.5 / 0.7.0 in Cargo.lock), the serde
// `T0Config` (config.rs:6-32), Weights::export_gguf (weights.rs:184-227) and
// cmd_export_gguf (crates/cli/src/main.rs:283-295).
//
// safetensors layout: u64 LE header length n, n bytes of JSON
//   {"<name>": {"dtype": "F32", "shape": [..], "data_offsets": [begin, end]},
//    "__metadata__": {..}}
// then the data buffer; offsets are relative to its start.  The checks are
// the crate's (header too small / too large, bad UTF-8 or JSON, tensors not
// laid end to end in offset order, a byte count that does not match the
// shape, a buffer not fully covered) plus weights.rs:127-129's F32-only rule.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>

#include "t0hip_internal.h"

namespace t0h {
namespace {

// ---- a small JSON reader (objects, arrays, strings, numbers, literals) ----
struct Json {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  double num = 0.0;
  bool integral = false;  // written without fraction or exponent
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;  // in file order
  const Json* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const char* p;
  const char* e;
  int code;
  const char* what;
  [[noreturn]] void fail(const std::string& msg) const { throw Error(code, std::string(what) + ": " + msg); }
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool eat(char c) {
    ws();
    if (p < e && *p == c) {
      ++p;
      return true;
    }
    return false;
  }
  void need(char c) {
    if (!eat(c)) fail(std::string("expected '") + c + "'");
  }
  static void put_utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) {
      s += (char)cp;
    } else if (cp < 0x800) {
      s += (char)(0xC0 | (cp >> 6));
      s += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += (char)(0xE0 | (cp >> 12));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    } else {
      s += (char)(0xF0 | (cp >> 18));
      s += (char)(0x80 | ((cp >> 12) & 0x3F));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    }
  }
  uint32_t hex4() {
    if (e - p < 4) fail("truncated \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0';
      else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
      else fail("bad \\u escape");
    }
    return v;
  }
  std::string string() {
    need('"');
    std::string s;
    while (true) {
      if (p >= e) fail("unterminated string");
      const char c = *p++;
      if (c == '"') return s;
      if ((unsigned char)c < 0x20) fail("control character in string");
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p >= e) fail("unterminated escape");
      const char x = *p++;
      switch (x) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {
            if (e - p < 2 || p[0] != '\\' || p[1] != 'u') fail("lone surrogate");
            p += 2;
            const uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            fail("lone surrogate");
          }
          put_utf8(s, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
  }
  Json value(int depth = 0) {
    if (depth > 64) fail("nesting too deep");
    ws();
    if (p >= e) fail("unexpected end");
    Json j;
    const char c = *p;
    if (c == '{') {
      ++p;
      j.kind = Json::OBJ;
      if (eat('}')) return j;
      do {
        ws();
        std::string k = string();
        need(':');
        j.obj.emplace_back(std::move(k), value(depth + 1));
      } while (eat(','));
      need('}');
    } else if (c == '[') {
      ++p;
      j.kind = Json::ARR;
      if (eat(']')) return j;
      do j.arr.push_back(value(depth + 1));
      while (eat(','));
      need(']');
    } else if (c == '"') {
      j.kind = Json::STR;
      j.str = string();
    } else if (e - p >= 4 && !std::memcmp(p, "true", 4)) {
      p += 4;
      j.kind = Json::BOOL;
      j.b = true;
    } else if (e - p >= 5 && !std::memcmp(p, "false", 5)) {
      p += 5;
      j.kind = Json::BOOL;
    } else if (e - p >= 4 && !std::memcmp(p, "null", 4)) {
      p += 4;
    } else if (c == '-' || (c >= '0' && c <= '9')) {
      const char* s = p;
      if (*p == '-') ++p;
      if (p >= e || *p < '0' || *p > '9') fail("bad number");
      if (*p == '0') ++p;
      else
        while (p < e && *p >= '0' && *p <= '9') ++p;
      bool integral = true;
      if (p < e && *p == '.') {
        integral = false;
        ++p;
        if (p >= e || *p < '0' || *p > '9') fail("bad number");
        while (p < e && *p >= '0' && *p <= '9') ++p;
      }
      if (p < e && (*p == 'e' || *p == 'E')) {
        integral = false;
        ++p;
        if (p < e && (*p == '+' || *p == '-')) ++p;
        if (p >= e || *p < '0' || *p > '9') fail("bad number");
        while (p < e && *p >= '0' && *p <= '9') ++p;
      }
      j.kind = Json::NUM;
      j.integral = integral;
      j.num = std::strtod(std::string(s, p).c_str(), nullptr);
    } else {
      fail("unexpected character");
    }
    return j;
  }
};

Json parse_json(const char* b, size_t n, int code, const char* what) {
  JsonParser ps{b, b + n, code, what};
  Json j = ps.value();
  ps.ws();
  if (ps.p != ps.e) ps.fail("trailing characters");
  return j;
}

bool valid_utf8(const uint8_t* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    const uint8_t c = s[i];
    size_t len = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
    if (!len || i + len > n) return false;
    for (size_t k = 1; k < len; ++k)
      if ((s[i + k] & 0xC0) != 0x80) return false;
    i += len;
  }
  return true;
}

uint64_t as_u64(const Json& j, const std::string& where) {
  if (j.kind != Json::NUM || !j.integral || j.num < 0 || j.num > 1.8e19)
    throw Error(T0H_ERR_SAFETENSORS, "safetensors: " + where + " must be a non-negative integer");
  return (uint64_t)j.num;
}

// ---- config.json as serde reads T0Config (config.rs:6-32) ----
ModelConfig config_from_json(const char* text) {
  if (!text) throw Error(T0H_ERR_INVALID_ARG, "config.json text is NULL");
  const Json j = parse_json(text, std::strlen(text), T0H_ERR_CONFIG, "config.json");
  if (j.kind != Json::OBJ) throw Error(T0H_ERR_CONFIG, "config.json: expected an object");
  auto req = [&](const char* k) -> const Json& {
    const Json* v = j.get(k);
    if (!v) throw Error(T0H_ERR_CONFIG, std::string("config.json: missing field `") + k + "`");
    return *v;
  };
  auto usize = [&](const char* k) -> uint32_t {  // usize fields: non-negative integers
    const Json& v = req(k);
    if (v.kind != Json::NUM || !v.integral || v.num < 0 || v.num > 4294967295.0)
      throw Error(T0H_ERR_CONFIG, std::string("config.json: `") + k + "` must be a non-negative integer");
    return (uint32_t)v.num;
  };
  auto f32 = [&](const Json& v, const std::string& k) -> float {
    if (v.kind != Json::NUM) throw Error(T0H_ERR_CONFIG, "config.json: `" + k + "` must be a number");
    return (float)v.num;  // serde_json reads the f64 and narrows it
  };
  ModelConfig mc;
  t0h_config& c = mc.c;
  c.embed_dim = usize("embed_dim");
  c.num_layers = usize("num_layers");
  c.num_heads = usize("num_heads");
  c.mlp_hidden_dim = usize("mlp_hidden_dim");
  c.patch_size = usize("patch_size");
  {
    const Json& g = req("group_every_n");
    if (g.kind != Json::NUM || !g.integral || std::fabs(g.num) > 9.2e18)
      throw Error(T0H_ERR_CONFIG, "config.json: `group_every_n` must be an integer");
    c.group_every_n = (int64_t)g.num;
  }
  c.dropout = f32(req("dropout"), "dropout");
  const Json& ql = req("quantile_levels");
  if (ql.kind != Json::ARR) throw Error(T0H_ERR_CONFIG, "config.json: `quantile_levels` must be an array");
  if (ql.arr.empty() || ql.arr.size() > T0H_MAX_QUANTILES)
    throw Error(T0H_ERR_UNSUPPORTED, "config.json: quantile_levels must hold 1.." + std::to_string(T0H_MAX_QUANTILES) +
                                         " levels");
  c.n_quantiles = (uint32_t)ql.arr.size();
  for (size_t i = 0; i < ql.arr.size(); ++i) c.quantile_levels[i] = f32(ql.arr[i], "quantile_levels");
  const Json* v;
  if ((v = j.get("scaler_use_arcsinh"))) {
    if (v->kind != Json::BOOL) throw Error(T0H_ERR_CONFIG, "config.json: `scaler_use_arcsinh` must be a boolean");
    c.scaler_use_arcsinh = v->b;
  } else {
    c.scaler_use_arcsinh = 1;  // config.rs:26-28
  }
  c.scaler_eps = (v = j.get("scaler_eps")) ? f32(*v, "scaler_eps") : 0.1f;  // config.rs:29-31
  if ((v = j.get("scaler_eps_mode"))) {
    if (v->kind != Json::STR) throw Error(T0H_ERR_CONFIG, "config.json: `scaler_eps_mode` must be a string");
    mc.eps_mode = v->str;
  } else {
    mc.eps_mode = "variance_offset";  // config.rs:32
  }
  c.scaler_variance_offset = mc.eps_mode != "std_clamp";  // scaler.rs:33
  return mc;
}

// ---- model.safetensors (F32 only, weights.rs:120-138) ----
std::vector<F32Tensor> read_safetensors(const uint8_t* b, size_t len) {
  auto bad = [](const std::string& m) { return Error(T0H_ERR_SAFETENSORS, "safetensors: " + m); };
  if (!b || len < 8) throw bad("header too small");
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | b[i];
  if (n > 100000000ull) throw bad("header too large");
  if (n > len - 8) throw bad("header length exceeds the file");
  const uint8_t* hdr = b + 8;
  if (!valid_utf8(hdr, (size_t)n)) throw bad("header is not valid UTF-8");
  const Json j = parse_json(reinterpret_cast<const char*>(hdr), (size_t)n, T0H_ERR_SAFETENSORS, "safetensors header");
  if (j.kind != Json::OBJ) throw bad("header is not a JSON object");
  const uint8_t* data = hdr + n;
  const size_t data_len = len - 8 - (size_t)n;
  struct Info {
    std::string name;
    std::string dtype;
    std::vector<size_t> shape;
    uint64_t begin, end;
  };
  std::vector<Info> infos;
  for (const auto& kv : j.obj) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != Json::OBJ) throw bad("__metadata__ must be an object");
      for (const auto& m : kv.second.obj)
        if (m.second.kind != Json::STR) throw bad("__metadata__ values must be strings");
      continue;
    }
    const Json& t = kv.second;
    const Json *dt = t.get("dtype"), *sh = t.get("shape"), *of = t.get("data_offsets");
    if (t.kind != Json::OBJ || !dt || !sh || !of || dt->kind != Json::STR || sh->kind != Json::ARR ||
        of->kind != Json::ARR || of->arr.size() != 2)
      throw bad("tensor " + kv.first + ": expected dtype, shape and two data_offsets");
    Info in{kv.first, dt->str, {}, as_u64(of->arr[0], kv.first + " data_offsets"),
            as_u64(of->arr[1], kv.first + " data_offsets")};
    for (const Json& d : sh->arr) in.shape.push_back((size_t)as_u64(d, kv.first + " shape"));
    infos.push_back(std::move(in));
  }
  // the crate's validation: tensors laid end to end in offset order, each
  // holding exactly its shape's bytes, covering the buffer
  std::vector<const Info*> order;
  for (const Info& in : infos) order.push_back(&in);
  std::stable_sort(order.begin(), order.end(), [](const Info* a, const Info* c) {
    return a->begin != c->begin ? a->begin < c->begin : a->end < c->end;
  });
  static const std::map<std::string, size_t> sizes = {
      {"BOOL", 1}, {"U8", 1}, {"I8", 1}, {"F8_E5M2", 1}, {"F8_E4M3", 1}, {"I16", 2}, {"U16", 2}, {"F16", 2},
      {"BF16", 2}, {"I32", 4}, {"U32", 4}, {"F32", 4}, {"F64", 8}, {"I64", 8}, {"U64", 8}};
  uint64_t at = 0;
  for (const Info* in : order) {
    auto sz = sizes.find(in->dtype);
    if (sz == sizes.end()) throw bad("tensor " + in->name + ": unknown dtype " + in->dtype);
    if (in->begin != at || in->end < in->begin) throw bad("tensor " + in->name + ": invalid data offsets");
    uint64_t count = 1;
    for (size_t d : in->shape) {
      if (d && count > UINT64_MAX / d) throw bad("tensor " + in->name + ": shape overflows");
      count *= d;
    }
    if (count > UINT64_MAX / sz->second || count * sz->second != in->end - in->begin)
      throw bad("tensor " + in->name + ": byte count does not match its shape and dtype");
    at = in->end;
  }
  if (at != data_len) throw bad("tensors do not cover the data buffer");
  std::vector<F32Tensor> out;
  for (const Info& in : infos) {
    if (in.dtype != "F32") throw Error(T0H_ERR_SAFETENSORS, "tensor " + in.name + " is " + in.dtype + ", expected F32");
    F32Tensor t{in.name, in.shape, std::vector<float>((size_t)((in.end - in.begin) / 4))};
    if (!t.data.empty()) std::memcpy(t.data.data(), data + in.begin, (size_t)(in.end - in.begin));  // little endian
    out.push_back(std::move(t));
  }
  return out;
}

}  // namespace

std::vector<uint8_t> export_gguf_from_safetensors(const uint8_t* st, size_t st_len, const char* config_json,
                                                  int quant) {
  if (quant != T0H_F32 && quant != T0H_F16 && quant != T0H_Q8_0 && quant != T0H_Q4_0)
    throw Error(T0H_ERR_INVALID_ARG, "export: quant must be F32, F16, Q8_0 or Q4_0");
  const ModelConfig mc = config_from_json(config_json);
  std::vector<F32Tensor> ts = read_safetensors(st, st_len);
  return write_gguf(meta_from_config(mc), plan_export(ts, quant));
}

}  // namespace t0h
