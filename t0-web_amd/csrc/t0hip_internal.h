// Internal host-side declarations shared by the t0hip library's translation units.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "t0hip.h"

namespace t0h {

constexpr int QK = 32;  // values per Q8_0/Q4_0 block (gguf.rs:18)

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

// ---- f16 (host) ----
float f16_to_f32(uint16_t h);
uint16_t f32_to_f16(float f);

// ---- codec ----
size_t row_bytes(int type, size_t n);  // 0 if invalid
void quantize(int type, const float* x, size_t n, uint8_t* out);
void dequantize(int type, const uint8_t* b, size_t n, float* out);

// ---- GGUF ----
enum { MV_U32 = 4, MV_F32 = 6, MV_BOOL = 7, MV_STRING = 8, MV_ARRAY = 9 };
struct MetaValue {
  int type = 0;
  uint32_t u32 = 0;
  float f32 = 0;
  bool b = false;
  std::string str;
  std::vector<float> arr;
};
struct GgufTensor {
  std::string name;
  std::vector<size_t> shape;  // row-major
  int type = 0;
  const uint8_t* data = nullptr;  // points into the caller's bytes
  size_t nbytes = 0;
  size_t n = 0;
};
struct GgufFile {
  std::map<std::string, MetaValue> meta;      // later keys replace earlier ones
  std::map<std::string, GgufTensor> tensors;  // later names replace earlier ones
};
GgufFile read_gguf(const uint8_t* bytes, size_t len);

struct TensorPlan {
  std::string name;
  std::vector<size_t> shape;
  int type;
  std::vector<uint8_t> data;
};
std::vector<uint8_t> write_gguf(const std::vector<std::pair<std::string, MetaValue>>& meta,
                                const std::vector<TensorPlan>& tensors);

struct ModelConfig {
  t0h_config c{};
  std::string eps_mode;
};
ModelConfig config_from_meta(const GgufFile& f);
std::vector<std::pair<std::string, MetaValue>> meta_from_config(const ModelConfig& mc);
// Layer pattern (config.rs:45-56): true = GROUP layer.  May be shorter than num_layers.
std::vector<bool> layer_types(const t0h_config& c);
// Checks that every tensor T0Model::load needs is present with a consistent shape.
void validate_model(const GgufFile& f, const t0h_config& c);
bool is_quantizable(const std::string& name);

// An F32 tensor as Weights holds one (weights.rs:21-23).
struct F32Tensor {
  std::string name;
  std::vector<size_t> shape;
  std::vector<float> data;
};
// weights.rs:187-227's export policy applied to `ts` (sorted by name in place).
std::vector<TensorPlan> plan_export(std::vector<F32Tensor>& ts, int quant);
// model.safetensors + config.json -> GGUF bytes (main.rs:283-295 cmd_export_gguf).
std::vector<uint8_t> export_gguf_from_safetensors(const uint8_t* st, size_t st_len, const char* config_json,
                                                  int quant);

// ---- error state ----
void set_error(const std::string& msg);

}  // namespace t0h
