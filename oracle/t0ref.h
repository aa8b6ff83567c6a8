/*
 * t0ref — CPU restatement of idle-intelligence/t0-web's t0-core ndarray path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity oracle and the CPU baseline
 * ("port") for the MI355X library in t0-web_amd/.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker; the product never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root).  The reference itself is Rust (t0-core on
 * burn-ndarray 0.20.1) and cannot be compiled in this environment, so this
 * restatement is pinned by the reference's own known-answer tests, an
 * independent numpy restatement of the quant codec, closed forms and
 * brute-force checks (see tests/).
 *
 * Parity unpinned (at the f32 rounding level only; every function below is
 * pinned to tolerance by a closed form or the float64 numpy forward):
 *   - t0r_linear's summation order.  The reference sums through
 *     matrixmultiply 0.3.11 (burn-ndarray 0.20.1 -> ndarray 0.17.2), which is
 *     absent here; this file uses a fixed 8-way split dot.
 *   - the f32 forms of silu, softplus and softmax inside t0r_forward (Burn
 *     0.20.1's are absent; the t0-fast WGSL forms silu_mul.wgsl:21,
 *     quantile_head.wgsl:19 and attention.wgsl:53-65 are restated), and the
 *     reduction order of the mean of squares in t0r_rmsnorm.
 *   - t0r_rope_tables' f64 pow/cos/sin (C libm here, Rust std there; at most
 *     one f64 ulp apart before the f32 cast).
 */
#ifndef T0REF_H
#define T0REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids, crates/t0-core/src/gguf.rs:31-49 */
enum { T0R_F32 = 0, T0R_F16 = 1, T0R_Q4_0 = 2, T0R_Q8_0 = 8 };

/* error codes (same numbering as the product's include/t0hip.h) */
enum {
  T0R_OK = 0,
  T0R_ERR_INVALID_ARG = -1,
  T0R_ERR_GGUF_MAGIC = -2,
  T0R_ERR_GGUF_VERSION = -3,
  T0R_ERR_GGUF_TENSOR_TYPE = -4,
  T0R_ERR_GGUF_META_TYPE = -5,
  T0R_ERR_GGUF_BOUNDS = -6,
  T0R_ERR_MISSING_TENSOR = -7,
  T0R_ERR_METADATA = -8,
  T0R_ERR_HORIZON = -9,
  T0R_ERR_FUTURE_ROWS = -10,
  T0R_ERR_SHAPE = -13,
  T0R_ERR_OOM = -15,
};

#define T0R_MAX_QUANTILES 64
#define T0R_MAX_HORIZON 1024 /* crates/t0-core/src/model.rs:26 */

typedef struct {
  uint32_t embed_dim, num_layers, num_heads, mlp_hidden_dim, patch_size;
  int64_t group_every_n;
  float dropout;
  uint32_t n_quantiles;
  float quantile_levels[T0R_MAX_QUANTILES];
  int32_t scaler_use_arcsinh;
  float scaler_eps;
  int32_t scaler_variance_offset; /* 1 = "variance_offset", 0 = "std_clamp" */
} t0r_config;

typedef struct t0r_model t0r_model;

/* ---- f16 (IEEE binary16, `half` 2.7.1 semantics) ---- */
float t0r_f16_to_f32(uint16_t h);
uint16_t t0r_f32_to_f16(float f);

/* ---- Q8_0 / Q4_0 block codec (gguf.rs:100-174) ---- */
size_t t0r_row_bytes(int ty, size_t n_elements);
void t0r_quantize_q8_0(const float* x, size_t n, uint8_t* out);
void t0r_dequantize_q8_0(const uint8_t* bytes, size_t n, float* out);
void t0r_quantize_q4_0(const float* x, size_t n, uint8_t* out);
void t0r_dequantize_q4_0(const uint8_t* bytes, size_t n, float* out);
int t0r_dequantize_for(int ty, const uint8_t* bytes, size_t n, float* out);
int t0r_quantize_for(int ty, const float* x, size_t n, uint8_t* out);

/* ---- model: GGUF load (dequantize-all-to-f32, weights.rs:151-163) ---- */
int t0r_model_load_gguf(const uint8_t* bytes, size_t len, t0r_model** out);
void t0r_model_free(t0r_model* m);
int t0r_model_config(const t0r_model* m, t0r_config* out);
/* f32 copy of a tensor; returns number of elements (0 if absent). shape may be NULL. */
size_t t0r_model_tensor(const t0r_model* m, const char* name, float* out, size_t cap, size_t shape[4], int* rank);
size_t t0r_model_tensor_count(const t0r_model* m);
/* GGUF export of the loaded f32 tensors (weights.rs:187-227). quant: T0R_F16/T0R_Q8_0/T0R_Q4_0
 * for the big matmuls (others F16), or T0R_F32 for an all-F32 file.  Returns byte count;
 * call with out=NULL to size. */
size_t t0r_export_gguf(const t0r_model* m, int quant, uint8_t* out, size_t cap);
void t0r_set_threads(int n);

/* ---- ops (ops.rs) ---- */
void t0r_linear(const float* x, const float* w, const float* b, float* y, size_t m, size_t k, size_t n, int relu);
void t0r_rmsnorm(const float* x, const float* scale, float* y, size_t rows, size_t dim, float eps);
void t0r_rope_tables(size_t seq_len, size_t head_dim, float* cos_t, float* sin_t, float* scale_t);
void t0r_quantile_head(const float* x, float* y, size_t rows, size_t n_q);
void t0r_interpolate_quantiles(const float* query, size_t nq, const float* levels, const float* values, size_t nl, float* out);
void t0r_weighted_quantile(const float* query, size_t nq, const float* weights, const float* samples, size_t ns, float* out);
void t0r_prob_mass(const float* levels, size_t n, float* out);

/* ---- host prep (data.rs, scaler.rs, mask.rs) on a [v,t] series ---- */
int t0r_scale_input(const float* variates, const int8_t* mask, const int64_t* group_ids, const int64_t* variate_type,
                    size_t v, size_t t, int use_arcsinh, float eps, int variance_offset,
                    float* scaled, float* loc, float* scale);
void t0r_build_time_mask(const int64_t* pg, const int64_t* pvt, const uint8_t* att, size_t v, size_t p, float* out);
void t0r_build_group_mask(const int64_t* pg, size_t v, size_t p, float* out);

/* ---- forward (model.rs:177-300): series already padded + scaled; out = [v, p, patch, n_q] ---- */
int t0r_forward(const t0r_model* m, size_t v, size_t t, const float* variates, const int8_t* mask,
                const int64_t* group_ids, const int64_t* variate_type,
                float* out, float* trace_patch_emb, float* trace_layer0);

/* ---- forecast drivers; out = [rows, horizon, n_q] ---- */
int t0r_forecast(const t0r_model* m, const float* ctx, size_t v, size_t t_ctx, size_t horizon, float* out);
int t0r_forecast_batch_chunked(const t0r_model* m, const float* ctx, size_t n_signals, size_t t_ctx, size_t horizon,
                               size_t chunk, float* out);
int t0r_forecast_batch_rows_chunked(const t0r_model* m, const float* ctx, const size_t* lengths, size_t n_signals,
                                    size_t horizon, size_t chunk, float* out);
int t0r_forecast_grouped(const t0r_model* m, const float* ctx, const int64_t* row_group, size_t n_rows, size_t t_ctx,
                         size_t horizon, float* out);
int t0r_forecast_grouped_ar(const t0r_model* m, const float* ctx, const int64_t* row_group, size_t n_rows,
                            size_t t_ctx, size_t horizon, size_t steps, float* out);
int t0r_forecast_rollout(const t0r_model* m, const float* ctx, size_t t_ctx, size_t prediction_length,
                         const float* query, size_t n_query, float* out);

#ifdef __cplusplus
}
#endif
#endif
