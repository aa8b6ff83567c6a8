// Fused element-wise / row kernels around the GEMMs: RMSNorm, on-device host
// prep (padding, causal scaler, patch encoder input, patch metadata), the
// quantile head with rescale + forecast slice, and the AR window update.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "kernels.h"
#include "lanes.h"
#include "t0hip_internal.h"

namespace t0h {
namespace {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(T0H_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// ---- RMSNorm (ops.rs:12-17; rmsnorm_full.wgsl): one wave per row ------------------
__global__ __launch_bounds__(256) void k_rmsnorm(const float* x, const float* scale, _Float16* out, const RowGather gth,
                                                 int rows, int dim) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* src = x + (size_t)gth.row(row) * dim;
  float ss = 0.0f;
  for (int c = lane * 4; c < dim; c += 256) {
    const float4 v = *reinterpret_cast<const float4*>(src + c);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
  const float denom = sqrtf(ss / (float)dim + 1e-8f);
  _Float16* dst = out + (size_t)row * dim;
  for (int c = lane * 4; c < dim; c += 256) {
    const float4 v = *reinterpret_cast<const float4*>(src + c);
    const float4 s = *reinterpret_cast<const float4*>(scale + c);
    const half4 h = {(_Float16)((v.x / denom) * s.x), (_Float16)((v.y / denom) * s.y), (_Float16)((v.z / denom) * s.z),
                     (_Float16)((v.w / denom) * s.w)};
    *reinterpret_cast<half4*>(dst + c) = h;
  }
}

// Rows up to 1024 wide: the wave holds its row and the scale in registers (one
// memory round trip), sums over DPP lane moves and row swaps, normalizes from
// registers.
__global__ __launch_bounds__(256) void k_rmsnorm_reg(const float* x, const float* scale, _Float16* out,
                                                     const RowGather gth, int rows, int dim) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* src = x + (size_t)gth.row(row) * dim;
  float4 v[4], g[4];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane * 4 + j * 256;
    v[j] = c < dim ? *reinterpret_cast<const float4*>(src + c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    g[j] = c < dim ? *reinterpret_cast<const float4*>(scale + c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
  }
  ss = rows_sum(lane_sum16(ss));
  const float denom = sqrtf(ss / (float)dim + 1e-8f);
  _Float16* dst = out + (size_t)row * dim;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = lane * 4 + j * 256;
    if (c < dim) {
      const float4 s = g[j];
      const half4 h = {(_Float16)((v[j].x / denom) * s.x), (_Float16)((v[j].y / denom) * s.y),
                       (_Float16)((v[j].z / denom) * s.z), (_Float16)((v[j].w / denom) * s.w)};
      *reinterpret_cast<half4*>(dst + c) = h;
    }
  }
}

// ---- forecast window (data.rs:52-155 + lib.rs:208-236) ------------------------------
// Rust 1.99 std f32::asinh: ln_1p(ax + ax / (hypot(1, 1/ax) + 1/ax)) with x's sign.
__device__ __forceinline__ float rust_asinh(float x) {
  const float ax = fabsf(x);
  const float ix = __fdiv_rn(1.0f, ax);
  return copysignf(log1pf(__fadd_rn(ax, __fdiv_rn(ax, __fadd_rn(hypotf(1.0f, ix), ix)))), x);
}

struct PatchAcc {
  int grp = -1, type = -1;
  bool found = false, any = false;
  __device__ void add(int mask, int group, int type_) {
    if (mask != T0H_MASK_PAD) {
      any = true;
      if (!found) {  // mask.rs:12-28: first non-PAD step's value
        found = true;
        grp = group;
        type = type_;
      }
    }
  }
};

__device__ __forceinline__ void write_patch_meta(const PatchOut& o, size_t m, const PatchAcc& a) {
  o.grp[m] = a.grp;
  o.type_raw[m] = a.type;
  o.type_idx[m] = a.type > 0 ? a.type : 0;  // model.rs:205 max(type, 0)
  o.att[m] = a.any ? 1 : 0;                 // mask.rs:32-43
}

// Welford state (count, mean, M2) and the pairwise merge of two disjoint
// segments (Chan, Golub & LeVeque), used to give each thread the exact running
// state at the start of its chunk.
struct Wf {
  float n, mean, m2;
};
__device__ __forceinline__ Wf wf_merge(Wf a, Wf b) {
  const float n = a.n + b.n;
  if (n == 0.0f) return a;
  const float delta = b.mean - a.mean;
  const float fb = b.n / n;
  return {n, a.mean + delta * fb, a.m2 + b.m2 + delta * delta * (a.n * fb)};
}

// One 256-thread workgroup per row: window construction (padding, NaN ->
// MISSING, ragged lead), the causal scaler (scaler.rs:44-118: Welford over VALID
// steps, emitted after each step's update, variance m2/(n-1), eps per mode, pad
// sentinel loc 0 / scale 1, then asinh), the patch encoder input [vals | k/ps |
// valid] (model.rs:185-197) and the patch metadata (mask.rs:12-43), with each
// patch's loc/scale at its last step for the rescale (scaler.rs:125-148).
// Each thread runs the reference's sequential Welford recurrence over its own
// chunk of steps, starting from the merged state of all earlier chunks.
__host__ __device__ inline size_t row_bytes(int t, int ps) {
  return ((size_t)(2 * t + 2 * (t / ps)) * 4 + (size_t)t + 255) / 256 * 256;
}

// The row's arrays live in the LDS (GM false) or, for windows too long for it,
// in the row's area of w.rows_mem (GM true); the same code runs on either.
template <bool GM>
__global__ __launch_bounds__(256) void k_prep_rows(const WindowDesc w, const PatchOut o) {
  extern __shared__ __align__(16) float psm[];
  __shared__ Wf st[2 * 256];  // scan buffers
  const int t = w.t, ps = w.ps, p = t / ps, r = blockIdx.x, tid = threadIdx.x;
  float* xs = GM ? reinterpret_cast<float*>(w.rows_mem + (size_t)r * row_bytes(t, ps)) : psm;  // [t] VALID value, NaN otherwise
  float* scv = xs + t;         // [t] scaled value
  float* pl = scv + t;         // [p] loc at patch end
  float* psc = pl + p;         // [p] scale at patch end
  // [t] step masks: the later passes read them here instead of rebuilding the
  // window (a dependent global load per step; one row's patch metadata loop
  // alone took about 20 us that way).  A step's group is the
  // row's and its type TARGET unless the step is PAD (group and type -1).
  unsigned char* smask = reinterpret_cast<unsigned char*>(psc + p);

  // Steps [0, pad_left) PAD | then t_ctx context steps: `lead` PAD (a ragged row
  // starts late), the row's values (NaN = MISSING) | the horizon WITHHELD
  // (data.rs:52-76, 110-155; lib.rs:215-216).  Eight steps a thread per batch,
  // their loads issued before any is used.
  {
    const int lead = w.t_ctx - w.len[r];
    const float* src = w.ctx + w.src_off[r] - lead - w.pad_left;  // value of step s at src[s]
    for (int b = tid; b < t; b += 256 * 8) {
      float xv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int s = b + 256 * u, c = s - w.pad_left;
        xv[u] = s < t && c >= lead && c < w.t_ctx ? src[s] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int s = b + 256 * u, c = s - w.pad_left;
        if (s >= t) break;
        int mk;
        if (c < 0 || (c < w.t_ctx && c < lead))
          mk = T0H_MASK_PAD;
        else if (c >= w.t_ctx)
          mk = T0H_MASK_WITHHELD;
        else
          mk = isnan(xv[u]) ? T0H_MASK_MISSING : T0H_MASK_VALID;
        xs[s] = mk == T0H_MASK_VALID ? xv[u] : NAN;
        smask[s] = (unsigned char)mk;
      }
    }
  }
  __syncthreads();
  const int C = (t + 255) / 256;
  const int s0 = min(t, tid * C), s1 = min(t, s0 + C);
  Wf loc_state{0.0f, 0.0f, 0.0f};
  for (int s = s0; s < s1; ++s) {
    const float x = xs[s];
    if (!isnan(x)) {
      loc_state.n += 1.0f;
      const float delta = x - loc_state.mean;
      loc_state.mean += delta / loc_state.n;
      loc_state.m2 += delta * (x - loc_state.mean);
    }
  }
  // inclusive scan of chunk states (Hillis-Steele, ping-pong)
  st[tid] = loc_state;
  __syncthreads();
  int cur = 0;
  for (int off = 1; off < 256; off <<= 1) {
    Wf v = st[cur * 256 + tid];
    if (tid >= off) v = wf_merge(st[cur * 256 + tid - off], v);
    st[(cur ^ 1) * 256 + tid] = v;
    cur ^= 1;
    __syncthreads();
  }
  Wf state = tid > 0 ? st[cur * 256 + tid - 1] : Wf{0.0f, 0.0f, 0.0f};
  for (int s = s0; s < s1; ++s) {
    const float x = xs[s];
    const bool valid = !isnan(x);
    if (valid) {
      state.n += 1.0f;
      const float delta = x - state.mean;
      state.mean += delta / state.n;
      state.m2 += delta * (x - state.mean);
    }
    const float var = state.n > 1.0f ? fmaxf(state.m2 / (state.n - 1.0f), 0.0f) : 0.0f;
    float sc = w.variance_offset ? sqrtf(var + w.eps) : fmaxf(sqrtf(var), w.eps);
    float lc = state.mean;
    if (smask[s] == T0H_MASK_PAD) {  // padding sentinel, group < 0 (scaler.rs:56-62)
      lc = 0.0f;
      sc = 1.0f;
    }
    const float z = __fdiv_rn(__fsub_rn(valid ? x : 0.0f, lc), sc);
    scv[s] = w.use_arcsinh ? rust_asinh(z) : z;
    if (s % ps == ps - 1) {
      pl[s / ps] = lc;
      psc[s / ps] = sc;
    }
  }
  __syncthreads();
  const size_t m0 = (size_t)r * p;
  _Float16* enc = o.enc_in + m0 * 3 * ps;
  const int F = 3 * ps, dq = 256 / F, dr = 256 % F;
  int pi = tid / F, f = tid % F;  // of idx, stepped by 256 without divisions
  for (int idx = tid; idx < p * F; idx += 256, pi += dq, f += dr) {
    if (f >= F) {
      f -= F;
      ++pi;
    }
    float val;
    if (f < ps)
      val = scv[pi * ps + f];
    else if (f < 2 * ps)
      val = (float)(f - ps) / (float)ps;
    else
      val = isnan(xs[pi * ps + f - 2 * ps]) ? 0.0f : 1.0f;
    enc[idx] = (_Float16)val;
  }
  const int g = w.group[r];
  for (int pi = tid; pi < p; pi += 256) {
    // every non-PAD step of the window has the row's group and type TARGET, so the
    // patch's first non-PAD step (mask.rs:12-28) gives those when there is one
    bool any = false;
#pragma unroll 8
    for (int k = 0; k < ps; ++k) any |= smask[pi * ps + k] != T0H_MASK_PAD;
    PatchAcc acc;
    if (any) acc.add(T0H_MASK_VALID, g, T0H_VT_TARGET);
    write_patch_meta(o, m0 + pi, acc);
    if (o.patch_loc) {
      o.patch_loc[m0 + pi] = pl[pi];
      o.patch_scale[m0 + pi] = psc[pi];
    }
    if (pi == 0) o.fut[r] = acc.type == T0H_VT_FUTURE ? 1 : 0;  // mask.rs:52
  }
}

}  // namespace

size_t prep_row_bytes(int t, int ps) { return row_bytes(t, ps); }
bool prep_fits_lds(int t, int ps) { return prep_row_bytes(t, ps) + 2 * 256 * sizeof(Wf) <= 160 * 1024; }

namespace {

__global__ __launch_bounds__(256) void k_series_patchify(const SeriesDev sd, const PatchOut o) {
  const int p = sd.t / sd.ps;
  const long long m = (long long)blockIdx.x * 256 + threadIdx.x;
  if (m >= (long long)sd.v * p) return;
  const int r = (int)(m / p), pi = (int)(m % p), ps = sd.ps;
  _Float16* enc = o.enc_in + m * 3 * ps;
  PatchAcc acc;
  for (int k = 0; k < ps; ++k) {
    const size_t src = (size_t)r * sd.t + pi * ps + k;
    const int mask = sd.mask[src];
    acc.add(mask, (int)sd.group_ids[src], (int)sd.variate_type[src]);
    enc[k] = (_Float16)sd.variates[src];
    enc[ps + k] = (_Float16)((float)k / (float)ps);
    enc[2 * ps + k] = (_Float16)(mask == T0H_MASK_VALID ? 1.0f : 0.0f);
  }
  write_patch_meta(o, m, acc);
}

// mask.rs:52: a row is FUTURE (bidirectional) when its first patch's reduced type is FUTURE.
__global__ void k_fut_rows(const int* type_raw, uint8_t* fut, int v, int p) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r < v) fut[r] = type_raw[(size_t)r * p] == T0H_VT_FUTURE ? 1 : 0;
}

// quantile_head.wgsl / ops.rs:195-210: q0 = raw0, q_i = q_{i-1} + log(1 + exp(raw_i))
__device__ __forceinline__ float softplus(float x) { return logf(1.0f + expf(x)); }

__global__ __launch_bounds__(256) void k_quantile_head(const float* dec, float* out, int rows, int ps, int nq) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long long)rows * ps) return;
  const float* src = dec + t * nq;
  float* dst = out + t * nq;
  float run = src[0];
  dst[0] = run;
  for (int i = 1; i < nq; ++i) {
    run = run + softplus(src[i]);
    dst[i] = run;
  }
}

// quantile head + rescale (scaler.rs:125-148) + forecast slice (lib.rs:75-96)
__global__ __launch_bounds__(256) void k_forecast_out(const ForecastOutDesc d) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long long)d.v * d.hp * d.ps) return;
  const int k = (int)(t % d.ps);
  const long long rh = t / d.ps;
  const int hh = (int)(rh % d.hp), r = (int)(rh / d.hp);
  const int step = hh * d.ps + k;
  if (step >= d.horizon) return;
  const size_t pm = (size_t)r * d.p + (d.ctx_p - 1 + hh);
  const float lc = d.patch_loc[pm], sc = d.patch_scale[pm];
  const float* src = d.dec + (size_t)rh * d.ps * d.nq + (size_t)k * d.nq;
  float* dst = d.out + ((size_t)r * d.horizon + step) * d.nq;
  float run = src[0];
  bool finite = true;
  for (int i = 0; i < d.nq; ++i) {
    finite = finite && isfinite(src[i]);
    if (i > 0) run = run + softplus(src[i]);
    const float u = d.use_arcsinh ? sinhf(run) : run;
    dst[i] = u * sc + lc;
  }
  if (!finite && d.nonfinite) *d.nonfinite = 1;
}

__global__ __launch_bounds__(256) void k_ar_shift(float* next, const float* ctx, const float* out, int v, int t_ctx,
                                                  int horizon, int nq, int q_idx) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long long)v * t_ctx) return;
  const int r = (int)(t / t_ctx), i = (int)(t % t_ctx);
  float x;
  if (horizon >= t_ctx) {
    x = out[((size_t)r * horizon + (horizon - t_ctx + i)) * nq + q_idx];
  } else if (i < t_ctx - horizon) {
    x = ctx[(size_t)r * t_ctx + i + horizon];
  } else {
    x = out[((size_t)r * horizon + (i - (t_ctx - horizon))) * nq + q_idx];
  }
  next[t] = x;
}

__global__ __launch_bounds__(256) void k_ar_store(float* dst, const float* src, int v, int horizon, int nq, int steps,
                                                  int step) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long per = (long long)horizon * nq;
  if (t >= (long long)v * per) return;
  const int r = (int)(t / per);
  const long long j = t % per;
  dst[(size_t)r * steps * per + (size_t)step * per + j] = src[t];
}

unsigned blocks(long long n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

// Device scratch of the no-allocation entry point.  In host code `scratch`
// names a host-side stand-in, never device memory: host code uses the address
// hipGetSymbolAddress returned for the current device (g_scratch[dev]).
static __device__ __align__(256) unsigned char scratch[T0H_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;
}  // namespace

void scratch_init() {
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) throw Error(T0H_ERR_UNSUPPORTED, "device id beyond the scratch table");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch[dev].load(std::memory_order_acquire)) return;
  void* ptr = nullptr;
  check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  if (!ptr) throw Error(T0H_ERR_HIP, "hipGetSymbolAddress(scratch) returned no address");
  g_scratch[dev].store(ptr, std::memory_order_release);
}

void* scratch_device_ptr(int dev) {
  void* ptr = dev >= 0 && dev < kMaxDevices ? g_scratch[dev].load(std::memory_order_acquire) : nullptr;
  if (!ptr) throw Error(T0H_ERR_INVALID_ARG, "no-allocation scratch not set up on device " + std::to_string(dev));
  return ptr;
}

void allow_dynamic_lds(const void* fn, std::atomic<uint64_t>& done) {
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  const uint64_t bit = 1ull << (dev & 63);
  if (done.load(std::memory_order_acquire) & bit) return;
  hipFuncAttributes fa;
  check_hip(hipFuncGetAttributes(&fa, fn), "hipFuncGetAttributes");
  const int cap = 160 * 1024 - (int)fa.sharedSizeBytes;
  check_hip(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, cap), "hipFuncSetAttribute");
  done.fetch_or(bit, std::memory_order_release);
}

void launch_rmsnorm(const float* x, const float* scale, _Float16* out, const RowGather& gth, int rows, int dim,
                    hipStream_t s) {
  if (rows <= 0) return;
  if (!x || !scale || !out) throw Error(T0H_ERR_INVALID_ARG, "rmsnorm: null pointer");
  if (dim <= 0 || dim % 4) throw Error(T0H_ERR_UNSUPPORTED, "rmsnorm: dim must be a positive multiple of 4");
  if (dim <= 1024)
    hipLaunchKernelGGL(k_rmsnorm_reg, dim3(blocks(rows, 4)), dim3(256), 0, s, x, scale, out, gth, rows, dim);
  else
    hipLaunchKernelGGL(k_rmsnorm, dim3(blocks(rows, 4)), dim3(256), 0, s, x, scale, out, gth, rows, dim);
  check_hip(hipGetLastError(), "k_rmsnorm launch");
}

void launch_window_prep(const WindowDesc& w, const PatchOut& o, hipStream_t s) {
  if (w.v <= 0) return;
  if (!w.ctx || !w.src_off || !w.len || !w.group) throw Error(T0H_ERR_INVALID_ARG, "prep: null window arrays");
  if (w.ps <= 0 || w.t % w.ps) throw Error(T0H_ERR_SHAPE, "prep: window not patch aligned");
  if (!o.enc_in || !o.grp || !o.att || !o.type_idx || !o.type_raw || !o.fut)
    throw Error(T0H_ERR_INVALID_ARG, "prep: null output arrays");
  if (prep_fits_lds(w.t, w.ps)) {
    static std::atomic<uint64_t> lds_set{0};
    allow_dynamic_lds(reinterpret_cast<const void*>(&k_prep_rows<false>), lds_set);
    hipLaunchKernelGGL(k_prep_rows<false>, dim3(w.v), dim3(256), prep_row_bytes(w.t, w.ps), s, w, o);
  } else {
    if (!w.rows_mem) throw Error(T0H_ERR_INVALID_ARG, "prep: long window without row memory");
    hipLaunchKernelGGL(k_prep_rows<true>, dim3(w.v), dim3(256), 0, s, w, o);
  }
  check_hip(hipGetLastError(), "k_prep_rows launch");
}

void launch_series_patchify(const SeriesDev& sd, const PatchOut& o, hipStream_t s) {
  if (sd.v <= 0) return;
  if (sd.ps <= 0 || sd.t % sd.ps) throw Error(T0H_ERR_SHAPE, "patchify: series not patch aligned");
  const long long n = (long long)sd.v * (sd.t / sd.ps);
  hipLaunchKernelGGL(k_series_patchify, dim3(blocks(n, 256)), dim3(256), 0, s, sd, o);
  check_hip(hipGetLastError(), "k_series_patchify launch");
}

void launch_fut_rows(const int* type_raw, uint8_t* fut, int v, int p, hipStream_t s) {
  if (v <= 0) return;
  hipLaunchKernelGGL(k_fut_rows, dim3(blocks(v, 256)), dim3(256), 0, s, type_raw, fut, v, p);
  check_hip(hipGetLastError(), "k_fut_rows launch");
}

void launch_quantile_head(const float* dec, float* out, int rows, int ps, int nq, hipStream_t s) {
  if (rows <= 0) return;
  hipLaunchKernelGGL(k_quantile_head, dim3(blocks((long long)rows * ps, 256)), dim3(256), 0, s, dec, out, rows, ps, nq);
  check_hip(hipGetLastError(), "k_quantile_head launch");
}

void launch_forecast_out(const ForecastOutDesc& d, hipStream_t s) {
  if (d.v <= 0 || d.hp <= 0) return;
  hipLaunchKernelGGL(k_forecast_out, dim3(blocks((long long)d.v * d.hp * d.ps, 256)), dim3(256), 0, s, d);
  check_hip(hipGetLastError(), "k_forecast_out launch");
}

void launch_ar_shift(float* ctx_next, const float* ctx, const float* out, int v, int t_ctx, int horizon, int nq,
                     int q_idx, hipStream_t s) {
  if (v <= 0 || t_ctx <= 0) return;
  hipLaunchKernelGGL(k_ar_shift, dim3(blocks((long long)v * t_ctx, 256)), dim3(256), 0, s, ctx_next, ctx, out, v, t_ctx,
                     horizon, nq, q_idx);
  check_hip(hipGetLastError(), "k_ar_shift launch");
}

void launch_ar_store(float* dst, const float* step_out, int v, int horizon, int nq, int steps, int step,
                     hipStream_t s) {
  if (v <= 0 || horizon <= 0) return;
  hipLaunchKernelGGL(k_ar_store, dim3(blocks((long long)v * horizon * nq, 256)), dim3(256), 0, s, dst, step_out, v,
                     horizon, nq, steps, step);
  check_hip(hipGetLastError(), "k_ar_store launch");
}

}  // namespace t0h
