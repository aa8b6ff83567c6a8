// Host-callable launchers for the CDNA4 (gfx950) kernels of the t0hip engine.
// Every launcher validates the shapes its kernel and grid assume before
// launching and throws t0h::Error on a violation.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>

namespace t0h {

// Raises kernel `fn`'s dynamic-LDS limit to everything the CU's 160 KB leaves
// after its static LDS, once per device: `done` holds one bit per device id
// (a static per kernel instantiation).  Launches still request only what they
// use; no launch calls hipFuncSetAttribute after the first one on a device.
void allow_dynamic_lds(const void* fn, std::atomic<uint64_t>& done);

// The no-allocation entry point's device scratch (a static __device__ array of
// T0H_NOALLOC_SCRATCH_BYTES): scratch_init() looks up its address on the
// current device once (call with that device current, at context creation);
// scratch_device_ptr(dev) returns it (throws if that device was never set up).
void scratch_init();
void* scratch_device_ptr(int dev);

// ---- quantized / f16 GEMM --------------------------------------------------
enum Epilogue {
  EPI_STORE_F32 = 0,  // y = acc + bias (+ row_add[row_add_idx[m]]) (relu opt.), f32 out
  EPI_STORE_F16 = 1,  // y = acc + bias (relu opt.), f16 out
  EPI_RESID_F32 = 2,  // y += acc + bias, f32 in/out (residual stream)
  EPI_SWIGLU_F16 = 3, // y[:, j] = silu(acc_j + b_j) * (acc_{H+j} + b_{H+j}), f16 out, N = H
};

struct GemmDesc {
  int wtype = 0;              // T0H_F16 / T0H_Q8_0 / T0H_Q4_0
  const void* w = nullptr;    // weight rows [N_w, K] in GGUF layout
  const void* a = nullptr;    // activations [M, K], row stride lda elements
  int a_f32 = 0;              // 1: a is float, 0: a is _Float16
  int lda = 0;
  const float* bias = nullptr;  // [N_w] or null
  void* y = nullptr;          // output, row stride ldy elements
  int ldy = 0;
  int M = 0, N = 0, K = 0;    // N = output columns (EPI_SWIGLU_F16: H; weight rows are 2H)
  int relu = 0;
  const float* row_add = nullptr;  // EPI_STORE_F32 only: [n_rows_table, N]
  const int* row_add_idx = nullptr;
  int epi = EPI_STORE_F32;
  // RMSNorm split across two GEMMs (rownorm_producer_ok / rownorm_consumer_ok).
  // Producer (EPI_RESID_F32): besides the new residual rows x, writes
  // norm_out[m, n] = f16(x[m, n] * norm_g[n] * RN_SCALE) (row stride N) and
  // norm_ssq[m, n / 32] = sum of x[m, n]^2 over each 32-column group.
  const float* norm_g = nullptr;
  _Float16* norm_out = nullptr;
  float* norm_ssq = nullptr;
  // Consumer (activations = a producer's norm_out): every output row is scaled
  // by 1 / (RN_SCALE * sqrt(sum of its ssq_parts partials / ssq_dim + 1e-8))
  // before the bias, which makes it the GEMM of the RMSNorm'd rows
  // (ops.rs:12-17: x / sqrt(mean(x^2) + eps) * scale).
  const float* row_ssq = nullptr;
  int ssq_parts = 0, ssq_dim = 0;
};
constexpr float RN_SCALE = 0.0625f;  // keeps unnormalized rows 16x further from the f16 range limit
// Whether the kernel launch_gemm picks for `d` can produce / consume the split RMSNorm.
bool rownorm_producer_ok(const GemmDesc& d);
bool rownorm_consumer_ok(const GemmDesc& d);

void launch_gemm(const GemmDesc& d, hipStream_t s);
// force = 0: pick by shape (M <= 16 small-M kernels; 16 < M < 1024 the split-K
// medium-M kernel up to 512 x 2304 outputs (F16 weights too); else MFMA tiles); 1: MFMA tile kernel (tile
// by shape); 2: small-M kernels; 3 / 4 / 5: MFMA kernel with 128x128 / 256x128 / 256x256
// tiles; 6: 256x256 DMA-fed kernel; 7 / 8: 256x256 / 256x128 kernels with
// register-dequantized weight fragments, 9 / 10: the 256x128 one with 192 / 128 rows (6-10:
// K % 64 == 0, f16 activations, quantized weights); FORCE_MID: medium-M kernel (quantized
// weights with K % 64 == 0, or F16 weights with K % 32 == 0 and K <= 2048).
constexpr int FORCE_MID = 32;
void launch_gemm_forced(const GemmDesc& d, int force, hipStream_t s);
void launch_dequant(int type, const void* w, size_t n, float* out, hipStream_t s);

// ---- norms -----------------------------------------------------------------
// out_f16[t] = x[gth.row(t)] / sqrt(mean(x^2) + 1e-8) * scale
// Rows a launch reads: row t itself, or (hp > 0, the forecast rows of a window)
// row (t / hp) * p + ctx_p - 1 + t % hp, patch ctx_p - 1 + h of window row t / hp.
struct RowGather {
  int p = 0, ctx_p = 0, hp = 0;
  __host__ __device__ int row(int t) const { return hp ? (t / hp) * p + ctx_p - 1 + t % hp : t; }
};
void launch_rmsnorm(const float* x, const float* scale, _Float16* out, const RowGather& gth, int rows, int dim,
                    hipStream_t s);

// ---- attention ---------------------------------------------------------------
struct AttnDesc {
  const _Float16* qkv = nullptr;  // [v*p, 3E]
  _Float16* out = nullptr;        // [v*p, E]
  int v = 0, p = 0, E = 0, heads = 0;
  const float* q_norm = nullptr;  // [head_dim] (group layers)
  const float* k_norm = nullptr;
  // time layers: per side [p, 128] = A | B with QK-norm scale, RoPE and xpos folded in:
  // rotated[e] = x[e] / rms(x) * A[e] + x[e^1] / rms(x) * B[e]  (xpos: scale on q, its recip on k)
  const float* rope_q = nullptr;
  const float* rope_k = nullptr;
  const int* grp = nullptr;          // [v*p] patch group id (-1 = all-PAD patch)
  const uint8_t* att = nullptr;      // [v*p] patch attendable
  const uint8_t* fut = nullptr;      // [v] row is FUTURE (bidirectional time attention)
  // group attention: rows of each row's group, as a permutation + per-row segment
  const int* perm = nullptr;         // [v]
  const int* seg_begin = nullptr;    // [v]
  const int* seg_len = nullptr;      // [v]
  int seg_max = 0;                   // longest segment (selects the kernel)
  const int* seg_start = nullptr;    // [n_seg] first permutation index of each segment
  int n_seg = 0;
  int qsplit = 1;                    // time attention: workgroups per (row, head), set by the launcher
  // time attention past T0H_LDS_PATCHES patches: workspace for the prepared keys
  // [v][heads][P32][64], the transposed values [v][heads][64][P32] and the key
  // groups [v][P32] (P32 = p rounded up to 32); null otherwise
  _Float16* kr = nullptr;
  _Float16* vt = nullptr;
  int* kg = nullptr;
};
// Longest window the single-pass (LDS-resident keys) time attention takes; longer
// windows stream their keys through workspace (AttnDesc kr / vt / kg).
constexpr int T0H_LDS_PATCHES = 256;
void launch_time_attention(const AttnDesc& d, hipStream_t s);
void launch_group_attention(const AttnDesc& d, hipStream_t s);

// ---- host-prep on device -------------------------------------------------------
// A forecast window (data.rs from_context/pad + lib.rs:208-236 ragged rows) described per row:
// steps [0,pad_left) PAD | [pad_left, pad_left+t_ctx): `lead` PAD then the row's `len` raw
// values (NaN = MISSING) | then horizon + right padding WITHHELD.
struct WindowDesc {
  const float* ctx = nullptr;        // raw values, flat
  const int64_t* src_off = nullptr;  // [v] offset of row r's first value in ctx
  const int* len = nullptr;          // [v] values of row r
  const int* group = nullptr;        // [v] row group id
  int v = 0, t_ctx = 0, horizon = 0, pad_left = 0, t = 0, ps = 0;
  int use_arcsinh = 1, variance_offset = 1;
  float eps = 0.1f;
  // windows whose per-row arrays exceed the LDS: one prep_row_bytes(t, ps) area per
  // row in device memory (null when the window fits the LDS)
  uint8_t* rows_mem = nullptr;
};
// Bytes of one row's prep arrays (values, scaled values, per-patch loc / scale,
// step masks), and whether they fit the LDS of one workgroup.
size_t prep_row_bytes(int t, int ps);
bool prep_fits_lds(int t, int ps);
struct PatchOut {
  _Float16* enc_in = nullptr;  // [v*p, 3*ps]
  int* grp = nullptr;          // [v*p]
  uint8_t* att = nullptr;      // [v*p]
  int* type_idx = nullptr;     // [v*p] max(type, 0)
  int* type_raw = nullptr;     // [v*p] reduced variate type (-1 = all PAD)
  uint8_t* fut = nullptr;      // [v]
  float* patch_loc = nullptr;  // [v*p] scaler loc at each patch's last step (may be null)
  float* patch_scale = nullptr;
};
// Window construction + causal scaler (scaler.rs:44-118) + patch encoder input and
// metadata, one workgroup per row.
void launch_window_prep(const WindowDesc& w, const PatchOut& o, hipStream_t s);
// Same from an explicit (already padded and scaled) series on device.
struct SeriesDev {
  const float* variates = nullptr;
  const int8_t* mask = nullptr;
  const int64_t* group_ids = nullptr;
  const int64_t* variate_type = nullptr;
  int v = 0, t = 0, ps = 0;
};
void launch_series_patchify(const SeriesDev& sd, const PatchOut& o, hipStream_t s);
void launch_fut_rows(const int* type_raw, uint8_t* fut, int v, int p, hipStream_t s);

// ---- outputs ---------------------------------------------------------------------
// Raw quantile head over rows x patch steps: out[r, k, q] (forward's [v,p,ps,nq]).
void launch_quantile_head(const float* dec, float* out, int rows, int ps, int nq, hipStream_t s);
// Forecast output: dec rows are (r, hp) pairs; applies the quantile head, sinh/rescale with
// the loc/scale of patch (ctx_p-1+hp) and writes out[r, hp*ps+k, q] for steps < horizon.
struct ForecastOutDesc {
  const float* dec = nullptr;  // [v*hp, ps*nq]
  const float* patch_loc = nullptr;
  const float* patch_scale = nullptr;
  float* out = nullptr;  // [v, horizon, nq]
  int* nonfinite = nullptr;  // set to 1 when a quantile logit is not finite (may be null)
  int v = 0, p = 0, ctx_p = 0, hp = 0, ps = 0, nq = 0, horizon = 0, use_arcsinh = 1;
};
void launch_forecast_out(const ForecastOutDesc& d, hipStream_t s);
// AR window update: ctx[r, :] <- (ctx[r, horizon:] ++ out[r, :, q_idx]) trailing t_ctx values.
void launch_ar_shift(float* ctx_next, const float* ctx, const float* out, int v, int t_ctx, int horizon, int nq,
                     int q_idx, hipStream_t s);
// Strided copy of one AR step's output into the [v, steps*horizon, nq] result.
void launch_ar_store(float* dst, const float* step_out, int v, int horizon, int nq, int steps, int step,
                     hipStream_t s);

}  // namespace t0h
