/*
 * t0hip.h — C ABI of the MI355X-native t0 quantized-inference engine.
 *
 * This is the boundary a Rust `t0-hip` crate (or any FFI) binds: plain C
 * types, host or device pointers plus sizes, int status codes, no exceptions
 * and no aborts across it.  Each entry point names the reference interface
 * it replaces (paths relative to idle-intelligence/t0-web):
 *
 *   t0h_ctx   ≡ t0_fast::Engine   (crates/t0-fast/src/engine.rs:18-44)
 *   t0h_model ≡ t0_fast::GpuModel (crates/t0-fast/src/model.rs:170-187)
 *
 * Threading: calls on one t0h_model are serialized by the caller (the
 * reference's "forward calls are sequential" contract, pool.rs:9-16); distinct
 * models may share one t0h_ctx and run concurrently, each on its own HIP
 * stream with its own workspace.
 *
 * Memory: host-pointer entry points copy in and out (outputs are written to
 * caller-owned buffers of the stated length).  Entry points suffixed `_dev`
 * take device pointers and run on the model's stream without host copies.
 */
#ifndef T0HIP_H
#define T0HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define T0H_ABI_VERSION 1
#define T0H_MAX_QUANTILES 64
#define T0H_MAX_HORIZON 1024 /* crates/t0-core/src/model.rs:26 MAX_HORIZON */
/* Longest window of t0h_forecast_grouped_dev_noalloc, in patches (the other entry
   points take any window that fits in device memory, like t0-core). */
#define T0H_NOALLOC_MAX_PATCHES 256
/* Device scratch of t0h_forecast_grouped_dev_noalloc, one per GPU (32 MiB). */
#define T0H_NOALLOC_SCRATCH_BYTES (32u << 20)

/* Status codes.  Each maps one reference failure (anyhow error or panic). */
enum t0h_status {
  T0H_OK = 0,
  T0H_ERR_INVALID_ARG = -1,      /* bad pointer/length; assert!s in lib.rs:195 */
  T0H_ERR_GGUF_MAGIC = -2,       /* gguf.rs:350-352 "not a GGUF file (bad magic)" */
  T0H_ERR_GGUF_VERSION = -3,     /* gguf.rs:353-356 unsupported GGUF version */
  T0H_ERR_GGUF_TENSOR_TYPE = -4, /* gguf.rs:41-49 unsupported ggml tensor type id */
  T0H_ERR_GGUF_META_TYPE = -5,   /* gguf.rs:281-283, 290 unsupported metadata value type */
  T0H_ERR_GGUF_BOUNDS = -6,      /* gguf.rs:397-400 tensor out of blob; truncated file */
  T0H_ERR_MISSING_TENSOR = -7,   /* weights.rs:268-270, t0-fast model.rs:255-257 */
  T0H_ERR_METADATA = -8,         /* weights.rs:70-97 missing/wrong-typed t0.* key; bad utf-8 */
  T0H_ERR_HORIZON = -9,          /* lib.rs:58-62 padded horizon > MAX_HORIZON */
  T0H_ERR_FUTURE_ROWS = -10,     /* scaler.rs:52-54 FUTURE covariate rows */
  T0H_ERR_NO_DEVICE = -11,       /* engine.rs:64-81 no GPU adapter */
  T0H_ERR_HIP = -12,             /* a HIP runtime call failed */
  T0H_ERR_SHAPE = -13,           /* tensor shape inconsistent with the config */
  T0H_ERR_UNSUPPORTED = -14,     /* outside this engine's documented limits */
  T0H_ERR_OOM = -15,             /* host or device allocation failed */
  T0H_ERR_SAFETENSORS = -16,     /* weights.rs:123-129 bad safetensors file or a non-F32 tensor */
  T0H_ERR_CONFIG = -17,          /* main.rs:285 config.json not a T0Config (serde_json error) */
  T0H_ERR_NUMERIC = -18,         /* no reference counterpart: a forecast's model outputs are not finite
                                    (an f16 activation beyond +-65504, or non-finite weights); the
                                    reference's f32 path would return them without an error */
};

/* ggml tensor type ids (gguf.rs:31-49) */
enum t0h_qtype { T0H_F32 = 0, T0H_F16 = 1, T0H_Q4_0 = 2, T0H_Q8_0 = 8 };

/* MaskType (data.rs:6-13) and VariateType (data.rs:15-20) */
enum { T0H_MASK_VALID = 0, T0H_MASK_PAD = 1, T0H_MASK_MISSING = 2, T0H_MASK_CENSORED = 3, T0H_MASK_WITHHELD = 4 };
enum { T0H_VT_TARGET = 0, T0H_VT_HISTORICAL = 1, T0H_VT_FUTURE = 2 };

/* ≡ T0Config (crates/t0-core/src/config.rs:6-22) */
typedef struct {
  uint32_t embed_dim, num_layers, num_heads, mlp_hidden_dim, patch_size;
  int64_t group_every_n;
  float dropout;
  uint32_t n_quantiles;
  float quantile_levels[T0H_MAX_QUANTILES];
  int32_t scaler_use_arcsinh;
  float scaler_eps;
  int32_t scaler_variance_offset; /* 1: "variance_offset", 0: "std_clamp" (scaler.rs:28-34) */
} t0h_config;

/* ≡ t0_core::data::TimeSeries (data.rs:24-33); all arrays row-major [v, t]. */
typedef struct {
  size_t v, t;
  const float* variates;
  const int8_t* mask;
  const int64_t* group_ids;
  const int64_t* variate_type;
} t0h_series;

typedef struct t0h_ctx t0h_ctx;
typedef struct t0h_model t0h_model;

/* ---- errors / version -------------------------------------------------- */
/* Message of the last failing call on this thread (≡ anyhow::Error's text). */
const char* t0h_last_error(void);
int t0h_abi_version(void);

/* ---- engine ------------------------------------------------------------ */
/* ≡ Engine::new_async (engine.rs:62-106).  T0H_ERR_NO_DEVICE when no GPU. */
int t0h_ctx_create(int device, t0h_ctx** out);
void t0h_ctx_destroy(t0h_ctx* ctx);

/* ---- model ------------------------------------------------------------- */
/* Parse and validate a GGUF (read_gguf gguf.rs:347-405 + config_from_gguf_metadata
 * weights.rs:69-112 + the tensor set T0Model::load needs, model.rs:108-147)
 * without touching a GPU.  cfg may be NULL. */
int t0h_gguf_inspect(const uint8_t* bytes, size_t len, t0h_config* cfg, size_t* n_tensors);

/* ≡ t0_fast::load_model_from_gguf (lib.rs:42-44 → GpuModel::load_from_gguf_bytes,
 * model.rs:302-348).  Q8_0/Q4_0 blocks are uploaded verbatim (llama.cpp AoS
 * layout) and stay resident; F16 matrices stay f16; F32 matrices are held as
 * f16; vectors (biases, norm scales, type embeddings) are held as f32. */
int t0h_model_load_gguf(t0h_ctx* ctx, const uint8_t* bytes, size_t len, t0h_model** out);
void t0h_model_destroy(t0h_model* model);
int t0h_model_config(const t0h_model* model, t0h_config* out);
/* ≡ GpuModel::quantizable_gpu_bytes / total_weight_bytes (model.rs:194-225) */
int t0h_model_weight_bytes(const t0h_model* model, uint64_t* quantizable, uint64_t* total);
/* The hipStream_t this model's work is issued on. */
void* t0h_model_stream(const t0h_model* model);
/* Device workspace currently held (≡ Pool::resident_bytes, pool.rs:64-66) and the
 * number of device allocations made since load (≡ Pool::alloc_count, pool.rs:51-57). */
int t0h_model_workspace(const t0h_model* model, uint64_t* resident_bytes, uint64_t* alloc_count);

/* Per-kernel-kind timing of this model's forward with HIP events on its stream
 * (no counterpart in the reference, which has no tracer: engine.rs:186-189 sets
 * timestamp_writes: None).  enable = 1 resets the counters and starts
 * recording; 0 stops.  Entries are indexed 0..n-1 in first-seen order; an index
 * past the end returns T0H_ERR_INVALID_ARG. */
int t0h_model_profile(t0h_model* model, int enable);
/* As t0h_model_profile(model, 1), but times only the launches of one kernel kind
 * (a name t0h_model_profile_entry reports), so that the events cost the forward
 * two records per launch of that kind and nothing elsewhere.  Stop with
 * t0h_model_profile(model, 0). */
int t0h_model_profile_kind(t0h_model* model, const char* kind);
int t0h_model_profile_entry(t0h_model* model, size_t i, char* name, size_t name_cap, uint64_t* launches,
                            double* total_ms);

/* Replay of the window forward as a HIP graph (no counterpart in the reference,
 * whose one-encoder, one-submit forward (t0-fast model.rs:693-808) is the
 * WebGPU analogue).  On by default: each forecast window's ~95 kernel launches
 * run eagerly the first time a window shape, input/output pointer pair and
 * workspace state is seen, are captured on the second and replayed after
 * that; off (enable = 0) every window runs eagerly.  Results are identical
 * either way.  While the profiler records events, windows run eagerly. */
int t0h_model_graph_replay(t0h_model* model, int enable);

/* Numeric guard (no counterpart in the reference, whose activations are f32).
 * The forward keeps its activations between kernels in f16; a value beyond
 * +-65504 there becomes inf and the forecast's outputs NaN.  Every forecast
 * records on the device whether any quantile logit was not finite.  The
 * host-output forecast entry points read that record with their results and
 * return T0H_ERR_NUMERIC (with the outputs written) when it is set; the
 * device-output ones (t0h_forecast_grouped_dev, _noalloc) do not wait, and
 * this call waits for the model's stream, returns T0H_ERR_NUMERIC if any
 * forecast since the last read was not finite, and clears the record. */
int t0h_model_check_numerics(t0h_model* model);

/* ---- forward ----------------------------------------------------------- */
/* ≡ model::forward_async (t0-fast model.rs:693-808) ≡ T0Model::forward (t0-core
 * model.rs:159-244): `series` already padded to whole patches and scaled.
 * out: [v, p, patch_size, n_quantiles] raw quantile-head output, p = t/patch.
 * trace_patch_emb / trace_layer0: optional [v, p, embed_dim] taps (model.rs:79-82). */
int t0h_forward(t0h_model* model, const t0h_series* series, float* out, size_t out_len, float* trace_patch_emb,
                float* trace_layer0);

/* ---- forecast entry points (outputs [rows, horizon, n_quantiles]) -------- */
/* ≡ t0_fast::forecast (lib.rs:102-109): v rows of one joint series (group 0). */
int t0h_forecast(t0h_model* model, const float* context, size_t v, size_t t_ctx, size_t horizon, float* out,
                 size_t out_len);
/* ≡ t0_fast::forecast_batch_chunked (lib.rs:118-146): independent univariate
 * signals, one group id each, chunk_size signals per forward (0 = one forward). */
int t0h_forecast_batch_chunked(t0h_model* model, const float* contexts, size_t n_signals, size_t t_ctx,
                               size_t horizon, size_t chunk_size, float* out, size_t out_len);
/* ≡ t0_fast::forecast_batch_rows_chunked (lib.rs:175-248): ragged contexts
 * concatenated per `lengths`. */
int t0h_forecast_batch_rows_chunked(t0h_model* model, const float* contexts, const size_t* lengths, size_t n_signals,
                                    size_t horizon, size_t chunk_size, float* out, size_t out_len);
/* Multivariate batch with an explicit group id per row (the 256 series x 3
 * variates workload).  The reference has no public entry point for this; it is
 * built from TimeSeries' pub fields the way lib.rs:208-236 builds its rows. */
int t0h_forecast_grouped(t0h_model* model, const float* contexts, const int64_t* row_group, size_t n_rows,
                         size_t t_ctx, size_t horizon, float* out, size_t out_len);
/* Same, device-resident: d_contexts [n_rows, t_ctx] and d_out [n_rows, horizon,
 * n_q] are device pointers; row_group is a host array.  Work is issued on the
 * model's stream; the call returns once it is enqueued (synchronize the stream
 * before reading d_out). */
int t0h_forecast_grouped_dev(t0h_model* model, const float* d_contexts, const int64_t* row_group, size_t n_rows,
                             size_t t_ctx, size_t horizon, float* d_out);
/* No counterpart in the reference: t0h_forecast_grouped_dev for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments and results; it calls no hipMalloc,
 * hipHostMalloc or hipFree.  The window's workspace is carved from one static
 * device array of T0H_NOALLOC_SCRATCH_BYTES per GPU (about 2,000 patch rows of
 * the 768-wide model: one 2048-step series is 66 rows), and its small host
 * metadata (group segments, RoPE tables) is staged through pinned memory the
 * model allocated at load.  A window that needs more scratch is rejected with
 * T0H_ERR_UNSUPPORTED before any work is issued.  Every no-allocation call on a
 * GPU shares that GPU's scratch, which keeps the last call's contents: calls
 * that overlap on one GPU (from different models, threads or streams) race.
 * Enqueued on the model's stream like the _dev entry point. */
int t0h_forecast_grouped_dev_noalloc(t0h_model* model, const float* d_contexts, const int64_t* row_group,
                                     size_t n_rows, size_t t_ctx, size_t horizon, float* d_out);
/* Autoregressive loop over t0h_forecast_grouped: after each step every row's
 * median-level quantile is appended and the window re-cut to the trailing
 * t_ctx values, weights staying resident.  out: [n_rows, steps*horizon, n_q]. */
int t0h_forecast_grouped_ar(t0h_model* model, const float* contexts, const int64_t* row_group, size_t n_rows,
                            size_t t_ctx, size_t horizon, size_t steps, float* out, size_t out_len);
/* ≡ t0_fast::forecast_rollout (lib.rs:259-341) ≡ t0_core::forecast_rollout
 * (model.rs:582-665): one univariate series; out [prediction_length, n_query]. */
int t0h_forecast_rollout(t0h_model* model, const float* context, size_t t_ctx, size_t prediction_length,
                         const float* query_levels, size_t n_query, float* out, size_t out_len);

/* ---- kernel-level entry points (device pointers, stream = hipStream_t or NULL) ----
 * The GEMM entry points take d_w, d_x and d_y 16-byte aligned (as hipMalloc returns
 * them) and d_bias 4-byte aligned; other pointers are refused with T0H_ERR_INVALID_ARG. */
/* Bit-exact dequantization ≡ dequantize_for (gguf.rs:213-226) on device. */
int t0h_dequant(int qtype, const void* d_blocks, size_t n_elements, float* d_out, void* stream);
/* ≡ t0-fast linear() (model.rs:406-504) / ops::linear (ops.rs:40-42):
 * d_y[m,n] = sum_k d_x[m,k] * W[n,k] + d_bias[n] (d_bias may be NULL), act 1 = relu.
 * W is [n, k] in GGUF layout of `wtype` (F16, Q8_0, Q4_0).  f32 in, f32 out. */
int t0h_gemm_q(int wtype, const void* d_w, const float* d_x, const float* d_bias, float* d_y, size_t m, size_t n,
               size_t k, int act, void* stream);
/* The forward's own GEMM kernels (f16 activations), exposed for kernel-level
 * parity tests and benchmarks.  d_x: f16 [m, k]; d_y: per epilogue
 *   0: f32 [m, n] = x W^T + b;  1: f16 [m, n] = x W^T + b;
 *   2: f32 [m, n] += x W^T + b (residual stream, model.rs:782-786);
 *   3: f16 [m, n] = silu(x W_g^T + b_g) * (x W_u^T + b_u), W with 2n rows gate
 *      first (ops.rs:57-61) — the fused SwiGLU of the FFN.
 * tile: 0 = as the forward picks, 1 = 128x128, 3 = 256x256, 4 = 256x256 with
 * DMA-fed activations (K % 128 == 0, quantized weights; falls back to 1),
 * 5 = 256x256 with the weights dequantized straight into MFMA operands,
 * 6 = the same with 256x128 tiles and two workgroups per CU, 7 / 8 = the
 * same with 192x128 / 128x128 tiles (5-8: K % 64 == 0, quantized weights;
 * fall back to 1). */
int t0h_gemm_f16(int wtype, const void* d_w, const void* d_x, const float* d_bias, void* d_y, size_t m, size_t n,
                 size_t k, int epilogue, int tile, void* stream);

/* ---- host codec, export, synthetic model -------------------------------- */
/* GgmlType::row_bytes (gguf.rs:61-70); 0 for an invalid count. */
size_t t0h_row_bytes(int qtype, size_t n_elements);
/* ≡ quantize_for (gguf.rs:192-211), host. */
int t0h_quantize(int qtype, const float* x, size_t n, uint8_t* out, size_t out_len);

typedef struct {
  t0h_config config;
  uint64_t seed;
  float weight_std;     /* rank-2 matrices ~ N(0, weight_std) */
  float bias_std;       /* biases ~ N(0, bias_std) */
  float norm_std;       /* norm scales ~ 1 + N(0, norm_std) */
  float emb_std;        /* type embeddings ~ N(0, emb_std) */
  float increment_bias; /* decoder output bias of quantile columns 1..n_q-1 */
} t0h_synth_spec;

/* Random-init model of the given config, written as GGUF the way
 * Weights::export_gguf (weights.rs:187-227) writes it: the four big per-layer
 * matmuls as `quant` (T0H_F16/T0H_Q8_0/T0H_Q4_0), everything else F16; quant =
 * T0H_F32 writes every tensor as F32.  Call with out = NULL to get *len. */
int t0h_synth_model_gguf(const t0h_synth_spec* spec, int quant, uint8_t* out, size_t cap, size_t* len);
/* Re-export a GGUF's tensors with another quantization (≡ export_gguf). */
int t0h_export_gguf(const uint8_t* bytes, size_t len, int quant, uint8_t* out, size_t cap, size_t* out_len);
/* ≡ t0-cli export-gguf (crates/cli/src/main.rs:283-295): Weights::load_bytes of
 * an all-F32 model.safetensors (weights.rs:115-140), the checkpoint's
 * config.json as serde reads T0Config (config.rs:6-32; NUL-terminated UTF-8),
 * then Weights::export_gguf (weights.rs:184-227) with quant T0H_F16, T0H_Q8_0 or
 * T0H_Q4_0 (T0H_F32 keeps every tensor F32).  Call with out = NULL to get
 * *out_len. */
int t0h_export_gguf_from_safetensors(const uint8_t* st_bytes, size_t st_len, const char* config_json, int quant,
                                     uint8_t* out, size_t cap, size_t* out_len);
/* ≡ t0_fast::load_model(engine, weights, config, quant) (crates/t0-fast/src/lib.rs:34-36):
 * the same export, loaded straight onto the device (T0H_F32 matrices are held
 * as f16 rows, as for an F32 GGUF). */
int t0h_model_load_safetensors(t0h_ctx* ctx, const uint8_t* st_bytes, size_t st_len, const char* config_json,
                               int quant, t0h_model** out);

#ifdef __cplusplus
}
#endif
#endif /* T0HIP_H */
