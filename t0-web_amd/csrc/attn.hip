// Attention for gfx950, reading the fused QKV activations in place.
//
// Semantics: ops.rs:153-190 (mhsa) with the masks of mask.rs:49-82 derived on
// the fly from per-patch metadata instead of dense [v,p,p] / [p,v,v] float
// masks:
//   time layers  — query patch i of variate row r attends key patch j iff
//                  (row is FUTURE or j <= i) and g_i >= 0 and g_j == g_i and
//                  patch j is attendable (mask.rs:49-65);
//   group layers — at a fixed patch, variate row a attends row b iff
//                  g_a >= 0 and g_b == g_a (mask.rs:69-82).
// A query whose every key is blocked gets the reference's result for an
// all-(-1e9) score row: exp(0) for every key, i.e. uniform weights over all
// keys of the row (time) or all variate rows (group).
// Per head: QK-RMSNorm (eps 1e-8) before RoPE (ops.rs:175-181), interleaved
// xPos RoPE on time layers (ops.rs:132-142; q scaled by the xpos table, k by
// its reciprocal), scores * 1/sqrt(head_dim), softmax, P*V.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "kernels.h"
#include "lanes.h"
#include "t0hip_internal.h"

namespace t0h {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int HD = 64;
constexpr int LDH = HD + 8;
constexpr int MAXKT = T0H_MAX_PATCHES / 16;

__host__ __device__ inline int round_up(int x, int m) { return (x + m - 1) / m * m; }

// V^T row stride in halfs: 8-byte aligned rows (half4 operand reads) whose
// dword stride is 2 (mod 4), so the key-pair dword writes of 8 dims x 8 key
// pairs land in distinct banks up to a 2-way conflict.
__host__ __device__ inline int vt_stride(int P32) { return P32 + 4; }

size_t time_attn_lds(int p) {
  const int P16 = round_up(p, 16), P32 = round_up(p, 32);
  return (size_t)(P16 + P32) * LDH * 2 + (size_t)HD * vt_stride(P32) * 2 + (size_t)P32 * 4 + (size_t)P32;
}


// One workgroup per (variate row, head), 4 waves over the 16-query tiles.
// Load phase: 8 lanes per 64-wide q/k row (16 B each), QK-RMSNorm reduced over
// the 8-lane group, interleaved xPos RoPE on the lane's 4 adjacent pairs, q/k
// stored row-major; v rows in key pairs, transposed into
// LDS as (key 2i, key 2i+1) dwords.  Compute phase: per 16-query tile,
// S^T = K Q^T and O = P V on v_mfma_f32_16x16x32_f16 with the tile's scores in
// registers; O is staged through the tile's own Q rows and stored in 16-byte
// row chunks.
template <int MAXKT>
__global__ __launch_bounds__(256) void k_time_attn(const AttnDesc d) {
  extern __shared__ __align__(16) _Float16 sm[];
  const int p = d.p, P16 = round_up(p, 16), P32 = round_up(p, 32), LDV = vt_stride(P32);
  _Float16* Qs = sm;
  _Float16* Ks = Qs + P16 * LDH;
  _Float16* Vt = Ks + P32 * LDH;
  int* Gk = reinterpret_cast<int*>(Vt + HD * LDV);
  uint8_t* Ak = reinterpret_cast<uint8_t*>(Gk + P32);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nth = blockDim.x, nwaves = nth >> 6;
  const int r = blockIdx.x / d.heads, h = blockIdx.x % d.heads;
  const int E = d.E, ld = 3 * E;
  const size_t row0 = (size_t)r * p;

  for (int i = tid; i < P32; i += nth) {
    Gk[i] = i < p ? d.grp[row0 + i] : -2;
    Ak[i] = i < p ? d.att[row0 + i] : 0;
  }
  // Items: q rows, k rows, v key pairs; each 8-lane group takes every 32nd.
  // All of a thread's global loads are issued before any is consumed.
  const int n_items = P16 + P32 + P32 / 2;
  const int d0 = (tid & 7) * 8;
  constexpr int NIT = (MAXKT * 16 * 5 / 2 + 31) / 32;  // items per group at the largest window
  uint4 g0[NIT], g1[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int item = (tid >> 3) + 32 * it;
    g0[it] = make_uint4(0, 0, 0, 0);
    g1[it] = make_uint4(0, 0, 0, 0);
    if (item >= n_items) continue;
    int which, i;
    if (item < P16) {
      which = 0;
      i = item;
    } else if (item < P16 + P32) {
      which = 1;
      i = item - P16;
    } else {
      which = 2;
      i = 2 * (item - P16 - P32);
    }
    const _Float16* src = d.qkv + (row0 + i) * ld + (size_t)which * E + h * HD + d0;
    if (i < p) g0[it] = *reinterpret_cast<const uint4*>(src);
    if (which == 2 && i + 1 < p) g1[it] = *reinterpret_cast<const uint4*>(src + ld);
  }
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int item = (tid >> 3) + 32 * it;
    if (item >= n_items) break;
    int which, i;
    if (item < P16) {
      which = 0;
      i = item;
    } else if (item < P16 + P32) {
      which = 1;
      i = item - P16;
    } else {
      which = 2;
      i = 2 * (item - P16 - P32);  // key pair (i, i+1)
    }
    const half8 hv = __builtin_bit_cast(half8, g0[it]);
    if (which == 2) {
      const half8 hw = __builtin_bit_cast(half8, g1[it]);
      uint32_t* vt2 = reinterpret_cast<uint32_t*>(Vt);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const half2v pr = {hv[e], hw[e]};
        vt2[((d0 + e) * LDV + i) >> 1] = __builtin_bit_cast(uint32_t, pr);
      }
      continue;
    }
    float x[8];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = (float)hv[e];
      ss += x[e] * x[e];
    }
    ss = lane_sum8(ss);
    half8 o = {};
    if (i < p) {
      const float inv = 1.0f / sqrtf(ss / (float)HD + 1e-8f);
      const float* nrm = (which ? d.k_norm : d.q_norm) + d0;
      const float* ct = d.rope_cos + (size_t)i * HD + d0;
      const float* st = d.rope_sin + (size_t)i * HD + d0;
      const float* xt = (which ? d.rope_scale_inv : d.rope_scale) + (size_t)i * HD + d0;
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (x[e] * inv) * nrm[e];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float rot = (e & 1) ? x[e - 1] : -x[e + 1];
        o[e] = (_Float16)(((x[e] * ct[e]) * xt[e]) + ((rot * st[e]) * xt[e]));
      }
    }
    *reinterpret_cast<uint4*>((which ? Ks : Qs) + i * LDH + d0) = __builtin_bit_cast(uint4, o);
  }
  __syncthreads();

  const bool fut = d.fut[r] != 0;
  const int nqt = P16 / 16, all_kt = P32 / 16;
  for (int qt = wave; qt < nqt; qt += nwaves) {
    const int q = qt * 16 + (lane & 15);
    const int gq = q < p ? Gk[q] : -1;
    const bool need_all = fut || __ballot(q < p && gq < 0) != 0;
    const int nkt = need_all ? all_kt : min(all_kt, (qt + 2) & ~1);
    const _Float16* qrow = Qs + (qt * 16 + (lane & 15)) * LDH + (lane >> 4) * 8;
    const half8 bq0 = *reinterpret_cast<const half8*>(qrow);
    const half8 bq1 = *reinterpret_cast<const half8*>(qrow + 32);

    float sc[MAXKT][4];
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < MAXKT; ++kt) {
      if (kt < nkt) {
        const _Float16* krow = Ks + (kt * 16 + (lane & 15)) * LDH + (lane >> 4) * 8;
        floatx4 s = {0.f, 0.f, 0.f, 0.f};
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const half8*>(krow), bq0, s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const half8*>(krow + 32), bq1, s, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = kt * 16 + (lane >> 4) * 4 + e;
          const bool ok = key < p && gq >= 0 && Gk[key] == gq && Ak[key] && (fut || key <= q);
          sc[kt][e] = ok ? s[e] * 0.125f : -INFINITY;
          mx = fmaxf(mx, sc[kt][e]);
        }
      }
    }
    mx = rows_max(mx);
    const bool uniform = mx == -INFINITY;
    float sum = 0.0f;
#pragma unroll
    for (int kt = 0; kt < MAXKT; ++kt) {
      if (kt < nkt) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = kt * 16 + (lane >> 4) * 4 + e;
          const float ev = uniform ? (key < p ? 1.0f : 0.0f) : __expf(sc[kt][e] - mx);
          sc[kt][e] = ev;
          sum += ev;
        }
      }
    }
    sum = rows_sum(sum);
    const float inv = 1.0f / sum;

    floatx4 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = (floatx4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < MAXKT / 2; ++c) {
      if (2 * c < nkt) {
        half8 pa;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pa[e] = (_Float16)(sc[2 * c][e] * inv);
          pa[4 + e] = (_Float16)(sc[2 * c + 1][e] * inv);
        }
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const _Float16* vrow = Vt + (dt * 16 + (lane & 15)) * LDV + 32 * c + (lane >> 4) * 4;
          const half4 lo = *reinterpret_cast<const half4*>(vrow);
          const half4 hi = *reinterpret_cast<const half4*>(vrow + 16);
          const half8 bv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, bv, o[dt], 0, 0, 0);
        }
      }
    }
    // Stage O (16 queries x 64 dims) in this tile's Q rows, which only this
    // wave reads, then write 16-byte row chunks.  LDS operations of one wave
    // complete in order.
    _Float16* ost = Qs + qt * 16 * LDH;
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) ost[((lane >> 4) * 4 + e) * LDH + dt * 16 + (lane & 15)] = (_Float16)o[dt][e];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int rr = c * 8 + (lane >> 3), cc = (lane & 7) * 8;
      const int qrow_i = qt * 16 + rr;
      if (qrow_i < p)
        *reinterpret_cast<uint4*>(d.out + (row0 + qrow_i) * E + h * HD + cc) = *reinterpret_cast<const uint4*>(ost + rr * LDH + cc);
    }
  }
}

// Group attention: 8 lanes per (query row, head), each lane owning 8 of the
// 64 dims; a wave covers 8 consecutive heads of a row, so every q/k/v load is
// one contiguous 1 KB span.  Keys are the query row's group (a segment of the
// group-sorted permutation); the norms and dot products reduce over the 8-lane
// group with DPP lane moves; online softmax.

__global__ __launch_bounds__(256) void k_group_attn(const AttnDesc d) {
  const int H = d.heads, E = d.E, p = d.p, v = d.v, ld = 3 * E;
  const long long task = ((long long)blockIdx.x * 256 + threadIdx.x) >> 3;
  const int sub = threadIdx.x & 7, d0 = sub * 8;
  if (task >= (long long)v * p * H) return;  // whole 8-lane groups exit together
  const int h = (int)(task % H);
  const long long m = task / H;
  const int r = (int)(m / p), pi = (int)(m % p);
  const int gq = d.grp[m];
  auto ld8 = [&](long long row, int which, float (&x)[8]) {
    const half8 hv = __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(d.qkv + row * ld + (size_t)which * E + h * HD + d0));
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (float)hv[e];
  };
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.0f;

  if (gq < 0) {  // all-PAD patch: every score is -1e9, uniform weights over all v rows
    for (int j = 0; j < v; ++j) {
      float vv[8];
      ld8((long long)j * p + pi, 2, vv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += vv[e];
    }
    const float inv = 1.0f / (float)v;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= inv;
  } else {
    float qn[8], kn[8];
    ld8(m, 0, qn);
#pragma unroll
    for (int e = 0; e < 8; ++e) kn[e] = d.k_norm[d0 + e];
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += qn[e] * qn[e];
    const float dq = sqrtf(lane_sum8(ss) / (float)HD + 1e-8f);
#pragma unroll
    for (int e = 0; e < 8; ++e) qn[e] = (qn[e] / dq) * d.q_norm[d0 + e];
    float mx = -INFINITY, l = 0.0f;
    const int b = d.seg_begin[r], n = d.seg_len[r];
    for (int idx = 0; idx < n; ++idx) {
      const int j = d.perm[b + idx];
      const long long mk = (long long)j * p + pi;
      if (d.grp[mk] != gq) continue;  // same value across the 8-lane group
      float kx[8], vx[8];
      ld8(mk, 1, kx);
      ld8(mk, 2, vx);
      float ks = 0.0f, dot = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ks += kx[e] * kx[e];
        dot += qn[e] * (kx[e] * kn[e]);
      }
      ks = lane_sum8(ks);
      dot = lane_sum8(dot);
      const float sc = (dot / sqrtf(ks / (float)HD + 1e-8f)) * 0.125f;
      const float nm = fmaxf(mx, sc);
      const float corr = __expf(mx - nm), pw = __expf(sc - nm);
      l = l * corr + pw;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = o[e] * corr + pw * vx[e];
      mx = nm;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= inv;
  }
  half8 hv;
#pragma unroll
  for (int e = 0; e < 8; ++e) hv[e] = (_Float16)o[e];
  *reinterpret_cast<uint4*>(d.out + m * E + h * HD + d0) = __builtin_bit_cast(uint4, hv);
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(T0H_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

void check_common(const AttnDesc& d) {
  if (!d.qkv || !d.out || !d.grp || !d.q_norm || !d.k_norm) throw Error(T0H_ERR_INVALID_ARG, "attention: null pointer");
  if (d.heads <= 0 || d.E != d.heads * HD)
    throw Error(T0H_ERR_UNSUPPORTED, "attention: head_dim must be 64 (embed_dim = 64 * num_heads)");
}

}  // namespace

void launch_time_attention(const AttnDesc& d, hipStream_t s) {
  if (d.v <= 0 || d.p <= 0) return;
  check_common(d);
  if (!d.att || !d.fut || !d.rope_cos || !d.rope_sin || !d.rope_scale || !d.rope_scale_inv)
    throw Error(T0H_ERR_INVALID_ARG, "time attention: null pointer");
  if (d.p > T0H_MAX_PATCHES)
    throw Error(T0H_ERR_UNSUPPORTED, "time attention: window of " + std::to_string(d.p) + " patches exceeds " +
                                         std::to_string(T0H_MAX_PATCHES));
  const size_t lds = time_attn_lds(d.p);
  const dim3 block(256);
  if (round_up(d.p, 32) / 16 <= 8) {
    check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_time_attn<8>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
              "hipFuncSetAttribute(k_time_attn)");
    hipLaunchKernelGGL(k_time_attn<8>, dim3(d.v * d.heads), block, lds, s, d);
  } else {
    check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_time_attn<MAXKT>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
              "hipFuncSetAttribute(k_time_attn)");
    hipLaunchKernelGGL(k_time_attn<MAXKT>, dim3(d.v * d.heads), block, lds, s, d);
  }
  check_hip(hipGetLastError(), "k_time_attn launch");
}

void launch_group_attention(const AttnDesc& d, hipStream_t s) {
  if (d.v <= 0 || d.p <= 0) return;
  check_common(d);
  if (!d.perm || !d.seg_begin || !d.seg_len) throw Error(T0H_ERR_INVALID_ARG, "group attention: null segment arrays");
  const long long lanes = (long long)d.v * d.p * d.heads * 8;
  hipLaunchKernelGGL(k_group_attn, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, s, d);
  check_hip(hipGetLastError(), "k_group_attn launch");
}

}  // namespace t0h
