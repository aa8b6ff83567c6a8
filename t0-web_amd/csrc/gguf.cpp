// GGUF v3 container, Q8_0/Q4_0 codec, export policy and the seeded synthetic
// model — the host-side format layer of the engine.
//
// Container semantics follow crates/t0-core/src/gguf.rs:228-405 (read_gguf /
// write_gguf): little-endian, ggml dimension order (ne[0] innermost, reversed
// to row-major on read), tensor offsets relative to a data blob that starts
// right after the tensor infos (unaligned in the file), 32-byte aligned offsets
// inside the blob.  Block codec follows gguf.rs:100-174 (llama.cpp's
// quantize_row_q8_0_ref / quantize_row_q4_0_ref layout).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>

#include "t0hip_internal.h"

namespace t0h {

// ---------------------------------------------------------------------------
// f16: the host compiler's _Float16 conversions are IEEE (exact widening,
// round-to-nearest-even narrowing) — the semantics of `half::f16` (2.7.1).
// ---------------------------------------------------------------------------
float f16_to_f32(uint16_t h) {
  _Float16 v;
  std::memcpy(&v, &h, 2);
  return static_cast<float>(v);
}
uint16_t f32_to_f16(float f) {
  _Float16 v = static_cast<_Float16>(f);
  uint16_t h;
  std::memcpy(&h, &v, 2);
  return h;
}

size_t row_bytes(int type, size_t n) {  // gguf.rs:61-70
  switch (type) {
    case T0H_F32: return n * 4;
    case T0H_F16: return n * 2;
    case T0H_Q8_0: return n % QK ? 0 : n / QK * (2 + QK);
    case T0H_Q4_0: return n % QK ? 0 : n / QK * (2 + QK / 2);
    default: return 0;
  }
}

namespace {
// Rust's `f as i32`: saturating, NaN -> 0.
int32_t sat_i32(float f) {
  if (std::isnan(f)) return 0;
  if (f >= 2147483647.0f) return std::numeric_limits<int32_t>::max();
  if (f <= -2147483648.0f) return std::numeric_limits<int32_t>::min();
  return static_cast<int32_t>(f);
}
void put_f16(uint8_t* o, float d) {
  uint16_t h = f32_to_f16(d);
  o[0] = uint8_t(h & 0xff);
  o[1] = uint8_t(h >> 8);
}
float get_f16(const uint8_t* o) { return f16_to_f32(uint16_t(o[0] | (o[1] << 8))); }
}  // namespace

void quantize(int type, const float* x, size_t n, uint8_t* out) {
  switch (type) {
    case T0H_F32: std::memcpy(out, x, n * 4); return;
    case T0H_F16:
      for (size_t i = 0; i < n; ++i) put_f16(out + 2 * i, x[i]);
      return;
    case T0H_Q8_0:  // gguf.rs:100-114: d = amax/127, q = round(x/d) clamped to i8
      for (size_t b = 0; b < n / QK; ++b) {
        const float* v = x + b * QK;
        uint8_t* o = out + b * (2 + QK);
        float amax = 0.0f;
        for (int i = 0; i < QK; ++i) amax = std::fmax(amax, std::fabs(v[i]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        put_f16(o, d);
        for (int i = 0; i < QK; ++i) {
          float r = std::round(v[i] * id);
          int8_t q = 0;
          if (!std::isnan(r)) q = static_cast<int8_t>(std::min(127.0f, std::max(-128.0f, r)));
          o[2 + i] = static_cast<uint8_t>(q);
        }
      }
      return;
    case T0H_Q4_0:  // gguf.rs:133-157: d = max/-8 (max = first value of largest |x|)
      for (size_t b = 0; b < n / QK; ++b) {
        const float* v = x + b * QK;
        uint8_t* o = out + b * (2 + QK / 2);
        float amax = 0.0f, mx = 0.0f;
        for (int i = 0; i < QK; ++i)
          if (std::fabs(v[i]) > amax) {
            amax = std::fabs(v[i]);
            mx = v[i];
          }
        const float d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        put_f16(o, d);
        for (int j = 0; j < QK / 2; ++j) {
          int32_t lo = std::clamp(sat_i32(std::floor(v[j] * id + 8.5f)), 0, 15);
          int32_t hi = std::clamp(sat_i32(std::floor(v[j + QK / 2] * id + 8.5f)), 0, 15);
          o[2 + j] = static_cast<uint8_t>(lo | (hi << 4));
        }
      }
      return;
  }
  throw Error(T0H_ERR_GGUF_TENSOR_TYPE, "unsupported quantization type " + std::to_string(type));
}

void dequantize(int type, const uint8_t* b, size_t n, float* out) {
  switch (type) {
    case T0H_F32: std::memcpy(out, b, n * 4); return;
    case T0H_F16:
      for (size_t i = 0; i < n; ++i) out[i] = get_f16(b + 2 * i);
      return;
    case T0H_Q8_0:  // gguf.rs:116-126
      for (size_t blk = 0; blk < n / QK; ++blk) {
        const uint8_t* o = b + blk * (2 + QK);
        const float d = get_f16(o);
        for (int i = 0; i < QK; ++i) out[blk * QK + i] = d * static_cast<float>(static_cast<int8_t>(o[2 + i]));
      }
      return;
    case T0H_Q4_0:  // gguf.rs:159-174
      for (size_t blk = 0; blk < n / QK; ++blk) {
        const uint8_t* o = b + blk * (2 + QK / 2);
        const float d = get_f16(o);
        for (int j = 0; j < QK / 2; ++j) {
          out[blk * QK + j] = d * (static_cast<float>(o[2 + j] & 0x0f) - 8.0f);
          out[blk * QK + j + QK / 2] = d * (static_cast<float>(o[2 + j] >> 4) - 8.0f);
        }
      }
      return;
  }
  throw Error(T0H_ERR_GGUF_TENSOR_TYPE, "unsupported tensor type " + std::to_string(type));
}

// ---------------------------------------------------------------------------
// Reader
// ---------------------------------------------------------------------------
namespace {
class Cursor {
 public:
  Cursor(const uint8_t* p, size_t n) : p_(p), n_(n) {}
  size_t pos() const { return pos_; }
  void need(size_t k, const char* what) const {
    if (k > n_ - pos_) throw Error(T0H_ERR_GGUF_BOUNDS, std::string("gguf: unexpected end of file reading ") + what);
  }
  template <typename T>
  T get(const char* what) {
    need(sizeof(T), what);
    T v;
    std::memcpy(&v, p_ + pos_, sizeof(T));
    pos_ += sizeof(T);
    return v;
  }
  std::string str(const char* what) {  // gguf.rs:234-239
    uint64_t len = get<uint64_t>(what);
    need(len, what);
    std::string s(reinterpret_cast<const char*>(p_ + pos_), len);
    pos_ += len;
    if (!utf8_ok(s)) throw Error(T0H_ERR_METADATA, "gguf string is not valid utf-8");
    return s;
  }

 private:
  static bool utf8_ok(const std::string& s) {
    size_t i = 0, n = s.size();
    while (i < n) {
      unsigned c = static_cast<unsigned char>(s[i]);
      int extra;
      uint32_t cp;
      if (c < 0x80) {
        ++i;
        continue;
      } else if ((c >> 5) == 0x6) {
        extra = 1;
        cp = c & 0x1f;
      } else if ((c >> 4) == 0xe) {
        extra = 2;
        cp = c & 0x0f;
      } else if ((c >> 3) == 0x1e) {
        extra = 3;
        cp = c & 0x07;
      } else {
        return false;
      }
      if (i + extra >= n) return false;
      for (int k = 1; k <= extra; ++k) {
        unsigned cc = static_cast<unsigned char>(s[i + k]);
        if ((cc >> 6) != 0x2) return false;
        cp = (cp << 6) | (cc & 0x3f);
      }
      static const uint32_t min_cp[4] = {0, 0x80, 0x800, 0x10000};
      if (cp < min_cp[extra] || cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) return false;
      i += extra + 1;
    }
    return true;
  }
  const uint8_t* p_;
  size_t n_;
  size_t pos_ = 0;
};
}  // namespace

GgufFile read_gguf(const uint8_t* bytes, size_t len) {  // gguf.rs:347-405
  Cursor c(bytes, len);
  if (len < 4 || std::memcmp(bytes, "GGUF", 4) != 0) throw Error(T0H_ERR_GGUF_MAGIC, "not a GGUF file (bad magic)");
  c.get<uint32_t>("magic");
  uint32_t version = c.get<uint32_t>("version");
  if (version != 3) throw Error(T0H_ERR_GGUF_VERSION, "unsupported GGUF version " + std::to_string(version) + ", expected 3");
  uint64_t n_tensors = c.get<uint64_t>("tensor count");
  uint64_t n_meta = c.get<uint64_t>("metadata count");
  if (n_tensors > len || n_meta > len) throw Error(T0H_ERR_GGUF_BOUNDS, "gguf: implausible tensor/metadata count");

  GgufFile f;
  for (uint64_t i = 0; i < n_meta; ++i) {  // gguf.rs:271-292
    std::string key = c.str("metadata key");
    MetaValue v;
    v.type = static_cast<int>(c.get<uint32_t>("metadata type"));
    switch (v.type) {
      case MV_U32: v.u32 = c.get<uint32_t>("u32"); break;
      case MV_F32: v.f32 = c.get<float>("f32"); break;
      case MV_BOOL: v.b = c.get<uint8_t>("bool") != 0; break;
      case MV_STRING: v.str = c.str("string"); break;
      case MV_ARRAY: {
        uint32_t et = c.get<uint32_t>("array type");
        uint64_t n = c.get<uint64_t>("array length");
        if (et != MV_F32)
          throw Error(T0H_ERR_GGUF_META_TYPE,
                      "gguf: only FLOAT32 arrays are supported by this reader, got type " + std::to_string(et));
        c.need(n * 4 / 4 == n ? n * 4 : ~size_t(0), "array");
        v.arr.resize(n);
        for (uint64_t k = 0; k < n; ++k) v.arr[k] = c.get<float>("array element");
        break;
      }
      default: throw Error(T0H_ERR_GGUF_META_TYPE, "gguf: unsupported metadata value type " + std::to_string(v.type));
    }
    f.meta[key] = std::move(v);
  }
  struct Info {
    GgufTensor t;
    uint64_t offset;
  };
  std::vector<Info> infos;
  infos.reserve(static_cast<size_t>(n_tensors));
  for (uint64_t i = 0; i < n_tensors; ++i) {
    Info in;
    in.t.name = c.str("tensor name");
    uint32_t nd = c.get<uint32_t>("n_dims");
    if (nd > 8) throw Error(T0H_ERR_SHAPE, "gguf: tensor " + in.t.name + " has too many dimensions");
    std::vector<size_t> ne(nd);
    for (uint32_t k = 0; k < nd; ++k) ne[k] = static_cast<size_t>(c.get<uint64_t>("dim"));
    in.t.shape.assign(ne.rbegin(), ne.rend());  // gguf.rs:381
    uint32_t ty = c.get<uint32_t>("tensor type");
    if (ty != T0H_F32 && ty != T0H_F16 && ty != T0H_Q4_0 && ty != T0H_Q8_0)
      throw Error(T0H_ERR_GGUF_TENSOR_TYPE, "unsupported ggml tensor type id " + std::to_string(ty));
    in.t.type = static_cast<int>(ty);
    in.offset = c.get<uint64_t>("tensor offset");
    infos.push_back(std::move(in));
  }
  const uint8_t* blob = bytes + c.pos();
  const size_t blob_len = len - c.pos();
  for (auto& in : infos) {
    size_t n = 1;
    for (size_t d : in.t.shape) n *= d;
    size_t nb = row_bytes(in.t.type, n);
    if (nb == 0 && n != 0)
      throw Error(T0H_ERR_SHAPE, "gguf: tensor " + in.t.name + " element count is not a multiple of 32");
    if (in.offset > blob_len || nb > blob_len - in.offset)
      throw Error(T0H_ERR_GGUF_BOUNDS, "gguf: tensor " + in.t.name + " out of bounds (" + std::to_string(in.offset) + ".." +
                                           std::to_string(in.offset + nb) + " of " + std::to_string(blob_len) +
                                           " byte blob)");
    in.t.n = n;
    in.t.nbytes = nb;
    in.t.data = blob + in.offset;
    f.tensors[in.t.name] = in.t;
  }
  return f;
}

// ---------------------------------------------------------------------------
// Writer (gguf.rs:299-345)
// ---------------------------------------------------------------------------
namespace {
struct Out {
  std::vector<uint8_t> b;
  template <typename T>
  void put(T v) {
    const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
    b.insert(b.end(), p, p + sizeof(T));
  }
  void str(const std::string& s) {
    put<uint64_t>(s.size());
    b.insert(b.end(), s.begin(), s.end());
  }
};
}  // namespace

std::vector<uint8_t> write_gguf(const std::vector<std::pair<std::string, MetaValue>>& meta,
                                const std::vector<TensorPlan>& tensors) {
  Out o;
  o.b.insert(o.b.end(), {'G', 'G', 'U', 'F'});
  o.put<uint32_t>(3);
  o.put<uint64_t>(tensors.size());
  o.put<uint64_t>(meta.size());
  for (const auto& kv : meta) {
    o.str(kv.first);
    const MetaValue& v = kv.second;
    o.put<uint32_t>(static_cast<uint32_t>(v.type));
    switch (v.type) {
      case MV_U32: o.put<uint32_t>(v.u32); break;
      case MV_F32: o.put<float>(v.f32); break;
      case MV_BOOL: o.put<uint8_t>(v.b ? 1 : 0); break;
      case MV_STRING: o.str(v.str); break;
      case MV_ARRAY:
        o.put<uint32_t>(MV_F32);
        o.put<uint64_t>(v.arr.size());
        for (float x : v.arr) o.put<float>(x);
        break;
      default: throw Error(T0H_ERR_GGUF_META_TYPE, "write_gguf: bad metadata type");
    }
  }
  std::vector<uint64_t> offsets;
  uint64_t cursor = 0;
  for (const auto& t : tensors) {
    offsets.push_back(cursor);
    cursor += t.data.size();
    if (cursor % 32) cursor += 32 - cursor % 32;
  }
  for (size_t i = 0; i < tensors.size(); ++i) {
    const auto& t = tensors[i];
    o.str(t.name);
    o.put<uint32_t>(static_cast<uint32_t>(t.shape.size()));
    for (auto it = t.shape.rbegin(); it != t.shape.rend(); ++it) o.put<uint64_t>(*it);
    o.put<uint32_t>(static_cast<uint32_t>(t.type));
    o.put<uint64_t>(offsets[i]);
  }
  uint64_t pos = 0;
  for (size_t i = 0; i < tensors.size(); ++i) {
    o.b.insert(o.b.end(), static_cast<size_t>(offsets[i] - pos), uint8_t(0));
    o.b.insert(o.b.end(), tensors[i].data.begin(), tensors[i].data.end());
    pos = offsets[i] + tensors[i].data.size();
  }
  return std::move(o.b);
}

// ---------------------------------------------------------------------------
// Config (weights.rs:69-112) and model tensor set (model.rs:84-147)
// ---------------------------------------------------------------------------
ModelConfig config_from_meta(const GgufFile& f) {
  auto get_u32 = [&](const char* k) -> uint32_t {
    auto it = f.meta.find(k);
    if (it == f.meta.end() || it->second.type != MV_U32)
      throw Error(T0H_ERR_METADATA, std::string("gguf: missing or wrong-typed metadata key ") + k);
    return it->second.u32;
  };
  auto find = [&](const char* k, int ty) -> const MetaValue* {
    auto it = f.meta.find(k);
    return (it != f.meta.end() && it->second.type == ty) ? &it->second : nullptr;
  };
  ModelConfig mc;
  t0h_config& c = mc.c;
  const MetaValue* ql = find("t0.quantile_levels", MV_ARRAY);
  c.embed_dim = get_u32("t0.embed_dim");
  c.num_layers = get_u32("t0.num_layers");
  c.num_heads = get_u32("t0.num_heads");
  c.mlp_hidden_dim = get_u32("t0.mlp_hidden_dim");
  c.patch_size = get_u32("t0.patch_size");
  c.group_every_n = static_cast<int64_t>(get_u32("t0.group_every_n"));
  if (!ql) throw Error(T0H_ERR_METADATA, "gguf: missing t0.quantile_levels metadata");
  if (ql->arr.empty() || ql->arr.size() > T0H_MAX_QUANTILES)
    throw Error(T0H_ERR_UNSUPPORTED, "gguf: t0.quantile_levels must hold 1.." + std::to_string(T0H_MAX_QUANTILES) + " levels");
  const MetaValue* v;
  c.dropout = (v = find("t0.dropout", MV_F32)) ? v->f32 : 0.0f;
  c.n_quantiles = static_cast<uint32_t>(ql->arr.size());
  std::copy(ql->arr.begin(), ql->arr.end(), c.quantile_levels);
  c.scaler_use_arcsinh = (v = find("t0.scaler_use_arcsinh", MV_BOOL)) ? v->b : 1;
  c.scaler_eps = (v = find("t0.scaler_eps", MV_F32)) ? v->f32 : 0.1f;
  mc.eps_mode = (v = find("t0.scaler_eps_mode", MV_STRING)) ? v->str : "variance_offset";
  c.scaler_variance_offset = mc.eps_mode != "std_clamp";
  return mc;
}

std::vector<std::pair<std::string, MetaValue>> meta_from_config(const ModelConfig& mc) {  // weights.rs:208-220
  const t0h_config& c = mc.c;
  auto U = [](uint32_t x) { MetaValue m; m.type = MV_U32; m.u32 = x; return m; };
  auto F = [](float x) { MetaValue m; m.type = MV_F32; m.f32 = x; return m; };
  MetaValue levels;
  levels.type = MV_ARRAY;
  levels.arr.assign(c.quantile_levels, c.quantile_levels + c.n_quantiles);
  MetaValue arcsinh;
  arcsinh.type = MV_BOOL;
  arcsinh.b = c.scaler_use_arcsinh != 0;
  MetaValue mode;
  mode.type = MV_STRING;
  mode.str = mc.eps_mode;
  return {{"t0.embed_dim", U(c.embed_dim)},
          {"t0.num_layers", U(c.num_layers)},
          {"t0.num_heads", U(c.num_heads)},
          {"t0.mlp_hidden_dim", U(c.mlp_hidden_dim)},
          {"t0.patch_size", U(c.patch_size)},
          {"t0.group_every_n", U(static_cast<uint32_t>(c.group_every_n))},
          {"t0.dropout", F(c.dropout)},
          {"t0.quantile_levels", levels},
          {"t0.scaler_use_arcsinh", arcsinh},
          {"t0.scaler_eps", F(c.scaler_eps)},
          {"t0.scaler_eps_mode", mode}};
}

std::vector<bool> layer_types(const t0h_config& c) {  // config.rs:45-56
  if (c.group_every_n <= 0) return std::vector<bool>(c.num_layers, false);
  size_t n = static_cast<size_t>(c.group_every_n);
  size_t total = (c.num_layers / n) * n;
  std::vector<bool> out(total);
  for (size_t i = 0; i < total; ++i) out[i] = (i % n) == n - 1;
  return out;
}

bool is_quantizable(const std::string& name) {  // weights.rs:32-37
  return name.find(".attention.wQKV.weight") != std::string::npos ||
         name.find(".attention.wO.weight") != std::string::npos || name.find(".mlp.0.weight") != std::string::npos ||
         name.find(".mlp.2.weight") != std::string::npos;
}

namespace {
void expect(const GgufFile& f, const std::string& name, std::vector<size_t> shape) {
  auto it = f.tensors.find(name);
  if (it == f.tensors.end()) throw Error(T0H_ERR_MISSING_TENSOR, "gguf: missing tensor " + name);
  if (it->second.shape != shape) {
    std::string s = "tensor " + name + " has shape [";
    for (size_t d : it->second.shape) s += std::to_string(d) + ",";
    s += "], expected [";
    for (size_t d : shape) s += std::to_string(d) + ",";
    throw Error(T0H_ERR_SHAPE, s + "]");
  }
}
}  // namespace

void validate_model(const GgufFile& f, const t0h_config& c) {
  if (c.num_heads == 0 || c.embed_dim == 0 || c.embed_dim % c.num_heads)
    throw Error(T0H_ERR_METADATA, "t0.embed_dim must be a positive multiple of t0.num_heads");
  if (c.patch_size == 0) throw Error(T0H_ERR_METADATA, "t0.patch_size must be positive");
  const size_t E = c.embed_dim, H = c.mlp_hidden_dim, hd = E / c.num_heads, ps = c.patch_size, nq = c.n_quantiles;
  // patch encoder / decoder residual blocks (model.rs:84-93); the hidden width is read from the file
  auto rblock = [&](const std::string& p, size_t in, size_t out) {
    auto it = f.tensors.find(p + ".mlp.hidden_layer.weight");
    if (it == f.tensors.end()) throw Error(T0H_ERR_MISSING_TENSOR, "gguf: missing tensor " + p + ".mlp.hidden_layer.weight");
    if (it->second.shape.size() != 2 || it->second.shape[1] != in)
      throw Error(T0H_ERR_SHAPE, "tensor " + p + ".mlp.hidden_layer.weight has the wrong shape");
    size_t hid = it->second.shape[0];
    expect(f, p + ".mlp.hidden_layer.bias", {hid});
    expect(f, p + ".mlp.output_layer.weight", {out, hid});
    expect(f, p + ".mlp.output_layer.bias", {out});
    expect(f, p + ".residual_layer.weight", {out, in});
    expect(f, p + ".residual_layer.bias", {out});
  };
  rblock("patch_encoder.projection", 3 * ps, E);
  auto te = f.tensors.find("patch_encoder.type_embeddings.weight");
  if (te == f.tensors.end()) throw Error(T0H_ERR_MISSING_TENSOR, "gguf: missing tensor patch_encoder.type_embeddings.weight");
  if (te->second.shape.size() != 2 || te->second.shape[1] != E || te->second.shape[0] == 0)
    throw Error(T0H_ERR_SHAPE, "tensor patch_encoder.type_embeddings.weight has the wrong shape");
  const size_t n_layers = layer_types(c).size();
  for (size_t i = 0; i < n_layers; ++i) {
    const std::string p = "transformer.layers." + std::to_string(i);
    expect(f, p + ".attention_block.norm.scale", {E});
    expect(f, p + ".attention_block.attention.wQKV.weight", {3 * E, E});
    expect(f, p + ".attention_block.attention.wQKV.bias", {3 * E});
    expect(f, p + ".attention_block.attention.wO.weight", {E, E});
    expect(f, p + ".attention_block.attention.wO.bias", {E});
    expect(f, p + ".attention_block.attention.q_norm.scale", {hd});
    expect(f, p + ".attention_block.attention.k_norm.scale", {hd});
    expect(f, p + ".norm.scale", {E});
    expect(f, p + ".mlp.0.weight", {2 * H, E});
    expect(f, p + ".mlp.0.bias", {2 * H});
    expect(f, p + ".mlp.2.weight", {E, H});
    expect(f, p + ".mlp.2.bias", {E});
  }
  expect(f, "transformer.out_norm.scale", {E});
  rblock("decoder", E, ps * nq);
}

}  // namespace t0h
