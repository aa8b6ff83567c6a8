// Seeded random-init t0 model, written as GGUF with the reference's export
// policy (crates/t0-core/src/weights.rs:187-227: tensors sorted by name, the
// four big per-layer matmuls quantized, every other tensor F16), plus
// re-export of an existing GGUF at another quantization.
//
// Tensor names and shapes are the ones T0Model::load reads
// (crates/t0-core/src/model.rs:84-147) plus `head.quantile_levels`, which the
// reference's checkpoints also carry.  The random source is the reference
// CLI's xorshift64 + Box-Muller generator (crates/cli/src/main.rs:313-330),
// seeded per tensor from (seed, tensor name) so values do not depend on the
// order tensors are generated in.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "t0hip_internal.h"

namespace t0h {
namespace {

struct Rng {  // crates/cli/src/main.rs:313-330
  uint64_t s;
  uint64_t next_u64() {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return s;
  }
  float uniform() { return static_cast<float>(next_u64() >> 40) / static_cast<float>(1ull << 24); }
  float normal() {
    float u1 = std::max(uniform(), 1e-7f);
    float u2 = uniform();
    return std::sqrt(-2.0f * std::log(u1)) * std::cos(2.0f * 3.14159265358979323846f * u2);
  }
};

uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
uint64_t fnv1a(const std::string& s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 0x100000001b3ull;
  }
  return h;
}

}  // namespace

// weights.rs:187-227's per-tensor policy: names sorted, the four big per-layer
// matmuls (rank 2, is_quantizable) as `quant`, every other tensor F16 (quant =
// F32 keeps everything F32).
std::vector<TensorPlan> plan_export(std::vector<F32Tensor>& ts, int quant) {
  std::sort(ts.begin(), ts.end(), [](const F32Tensor& a, const F32Tensor& b) { return a.name < b.name; });
  std::vector<TensorPlan> plans;
  for (auto& t : ts) {
    int ty;
    if (quant == T0H_F32)
      ty = T0H_F32;
    else
      ty = (t.shape.size() == 2 && is_quantizable(t.name)) ? quant : T0H_F16;  // weights.rs:195-199
    size_t nb = row_bytes(ty, t.data.size());
    if (nb == 0 && !t.data.empty()) throw Error(T0H_ERR_SHAPE, "tensor " + t.name + " cannot be quantized as requested");
    TensorPlan p{t.name, t.shape, ty, std::vector<uint8_t>(nb)};
    quantize(ty, t.data.data(), t.data.size(), p.data.data());
    plans.push_back(std::move(p));
  }
  return plans;
}

std::vector<uint8_t> synth_model_gguf(const t0h_synth_spec& s, int quant) {
  const t0h_config& c = s.config;
  if (c.num_heads == 0 || c.embed_dim % c.num_heads || c.patch_size == 0 || c.n_quantiles == 0 ||
      c.n_quantiles > T0H_MAX_QUANTILES)
    throw Error(T0H_ERR_INVALID_ARG, "synth: inconsistent config");
  if (quant != T0H_F32 && quant != T0H_F16 && quant != T0H_Q8_0 && quant != T0H_Q4_0)
    throw Error(T0H_ERR_INVALID_ARG, "synth: quant must be F32, F16, Q8_0 or Q4_0");
  const size_t E = c.embed_dim, H = c.mlp_hidden_dim, hd = E / c.num_heads, ps = c.patch_size, nq = c.n_quantiles;
  std::vector<F32Tensor> ts;
  auto add = [&](const std::string& name, std::vector<size_t> shape) {
    size_t n = 1;
    for (size_t d : shape) n *= d;
    F32Tensor t{name, shape, std::vector<float>(n)};
    Rng rng{splitmix64(s.seed ^ fnv1a(name)) | 1};
    const bool is_bias = name.size() > 5 && name.compare(name.size() - 5, 5, ".bias") == 0;
    const bool is_scale = name.size() > 6 && name.compare(name.size() - 6, 6, ".scale") == 0;
    const bool is_emb = name.find("type_embeddings") != std::string::npos;
    for (size_t i = 0; i < n; ++i) {
      float z = rng.normal();
      if (is_scale)
        t.data[i] = 1.0f + s.norm_std * z;
      else if (is_bias)
        t.data[i] = s.bias_std * z;
      else if (is_emb)
        t.data[i] = s.emb_std * z;
      else
        t.data[i] = s.weight_std * z;
    }
    // Quantile increments (columns 1..n_q-1 of each patch step) get a shared
    // offset so the cumulative-softplus head starts from narrow quantile spreads.
    if (name == "decoder.mlp.output_layer.bias")
      for (size_t i = 0; i < n; ++i)
        if (i % nq != 0) t.data[i] += s.increment_bias;
    ts.push_back(std::move(t));
  };
  auto rblock = [&](const std::string& p, size_t in, size_t hid, size_t out) {
    add(p + ".mlp.hidden_layer.weight", {hid, in});
    add(p + ".mlp.hidden_layer.bias", {hid});
    add(p + ".mlp.output_layer.weight", {out, hid});
    add(p + ".mlp.output_layer.bias", {out});
    add(p + ".residual_layer.weight", {out, in});
    add(p + ".residual_layer.bias", {out});
  };
  rblock("patch_encoder.projection", 3 * ps, E, E);
  add("patch_encoder.type_embeddings.weight", {3, E});
  for (size_t i = 0; i < c.num_layers; ++i) {
    const std::string p = "transformer.layers." + std::to_string(i);
    add(p + ".attention_block.norm.scale", {E});
    add(p + ".attention_block.attention.wQKV.weight", {3 * E, E});
    add(p + ".attention_block.attention.wQKV.bias", {3 * E});
    add(p + ".attention_block.attention.wO.weight", {E, E});
    add(p + ".attention_block.attention.wO.bias", {E});
    add(p + ".attention_block.attention.q_norm.scale", {hd});
    add(p + ".attention_block.attention.k_norm.scale", {hd});
    add(p + ".norm.scale", {E});
    add(p + ".mlp.0.weight", {2 * H, E});
    add(p + ".mlp.0.bias", {2 * H});
    add(p + ".mlp.2.weight", {E, H});
    add(p + ".mlp.2.bias", {E});
  }
  add("transformer.out_norm.scale", {E});
  rblock("decoder", E, E, ps * nq);
  F32Tensor lv{"head.quantile_levels", {nq}, std::vector<float>(c.quantile_levels, c.quantile_levels + nq)};
  ts.push_back(std::move(lv));

  ModelConfig mc;
  mc.c = c;
  mc.eps_mode = c.scaler_variance_offset ? "variance_offset" : "std_clamp";
  return write_gguf(meta_from_config(mc), plan_export(ts, quant));
}

std::vector<uint8_t> export_gguf(const uint8_t* bytes, size_t len, int quant) {
  if (quant != T0H_F32 && quant != T0H_F16 && quant != T0H_Q8_0 && quant != T0H_Q4_0)
    throw Error(T0H_ERR_INVALID_ARG, "export: quant must be F32, F16, Q8_0 or Q4_0");
  GgufFile f = read_gguf(bytes, len);
  ModelConfig mc = config_from_meta(f);
  std::vector<F32Tensor> ts;
  for (const auto& kv : f.tensors) {  // Weights::load_gguf_bytes dequantizes everything (weights.rs:154-159)
    F32Tensor t{kv.first, kv.second.shape, std::vector<float>(kv.second.n)};
    dequantize(kv.second.type, kv.second.data, kv.second.n, t.data.data());
    ts.push_back(std::move(t));
  }
  return write_gguf(meta_from_config(mc), plan_export(ts, quant));
}

}  // namespace t0h
