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
constexpr int TA_WAVES = 4;

__host__ __device__ inline int round_up(int x, int m) { return (x + m - 1) / m * m; }

// V^T row stride in halfs: 8-byte aligned rows (half4 operand reads) whose
// dword stride is 2 (mod 4), so the key-pair dword writes of 8 dims x 8 key
// pairs land in distinct banks up to a 2-way conflict.
__host__ __device__ inline int vt_stride(int P32) { return P32 + 4; }

// LDS of one (row, head) workgroup: Ks [P16 + 1][LDH] f16 keys after norm + RoPE
// (rows >= p zero; row P16 takes the key items past the window) | Vt [HD][LDV] f16 values by key pairs (keys >= p zero) |
// Os [TA_WAVES][16][LDH] per-wave output staging | Kg [P32] int key group if
// attendable, -2 if not, -4 past the window.
size_t time_attn_lds(int p) {
  const int P16 = round_up(p, 16), P32 = round_up(p, 32);
  return (size_t)(P16 + 1) * LDH * 2 + (size_t)HD * vt_stride(P32) * 2 + (size_t)TA_WAVES * 16 * LDH * 2 + (size_t)P32 * 4;
}

__device__ __forceinline__ void unpack8(uint4 u, float* x) {
  const half8 hv = __builtin_bit_cast(half8, u);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (float)hv[e];
}

// Eight adjacent dims (four rotation pairs) of a QK-normalized, rotated row:
// inv * (x[e] * A[e] + x[e^1] * B[e]) with A at tab[0..7] and B at tab[64..71].
__device__ __forceinline__ half8 rotate8(const float* x, const float* a, const float* b, float inv) {
  half8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (_Float16)(((x[e] * inv) * a[e]) + ((x[e ^ 1] * inv) * b[e]));
  return o;
}

__device__ __forceinline__ void load_f8(const float* t, float* a) {
  const float4 u = *reinterpret_cast<const float4*>(t), w = *reinterpret_cast<const float4*>(t + 4);
  a[0] = u.x, a[1] = u.y, a[2] = u.z, a[3] = u.w, a[4] = w.x, a[5] = w.y, a[6] = w.z, a[7] = w.w;
}

// One workgroup (qsplit of them for few rows) per (variate row, head), TA_WAVES waves.
// Key phase: 8 lanes per 64-wide k row (16 B each), QK-RMSNorm reduced over
// the 8-lane group, norm scale + interleaved xPos RoPE from the folded tables,
// keys stored row-major; v rows in key pairs, transposed into LDS as
// (key 2i, key 2i+1) dwords.  Query phase: each wave takes 16-query tiles in a
// snake order over decreasing causal cost; a tile's queries are loaded straight
// into the MFMA operand layout (lane: query lane%16, dims 8(lane/16)..+7 and
// 32 + 8(lane/16)..+7), normalized across the four lanes that hold a query and
// rotated in registers; S^T = K Q^T and O = P V on v_mfma_f32_16x16x32_f16 with
// the tile's scores in registers; O is staged through the wave's LDS region and
// stored in 16-byte row chunks.
//
// LAT (few (row, head) pairs, so the chain of memory round trips of one
// workgroup is the kernel's time): rows past the window are loaded from a
// clamped row and discarded where used instead of skipped under a branch, and
// the key tables are prefetched two items ahead, so a workgroup waits about
// once before its barrier.  With many pairs the other workgroups on the CU hide
// those round trips and the extra loads would only cost issue slots.
template <int MAXKT, bool LAT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MAXKT <= 8 ? 4 : 3))) void k_time_attn(const AttnDesc d) {
  extern __shared__ __align__(16) _Float16 sm[];
  const int p = d.p, P16 = round_up(p, 16), P32 = round_up(p, 32), LDV = vt_stride(P32);
  _Float16* Ks = sm;
  _Float16* Vt = Ks + (P16 + 1) * LDH;  // Ks row P16: where key items past the window are written
  _Float16* Os = Vt + HD * LDV;
  int* Kg = reinterpret_cast<int*>(Os + TA_WAVES * 16 * LDH);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, part = lane >> 4;
  // qsplit workgroups share a (row, head): each loads every key and takes every
  // qsplit-th wave slot of the query tiles
  const int S = d.qsplit, sp = blockIdx.x % S, rh = blockIdx.x / S;
  const int r = rh / d.heads, h = rh % d.heads;
  const int NW = TA_WAVES * S, wv = wave * S + sp;
  const int E = d.E, ld = 3 * E;
  const size_t row0 = (size_t)r * p;
  const _Float16* qb = d.qkv + row0 * ld + h * HD;  // q; k at +E, v at +2E
  const int nqt = P16 / 16, all_kt = P32 / 16;

  // This wave's j-th tile in cost order (the snake over waves); -1 when past the last.
  auto tile_at = [&](int k) {
    const int j = (k >> 1) * 2 * NW + ((k & 1) ? 2 * NW - 1 - wv : wv);
    return j < nqt ? nqt - 1 - j : -1;
  };
  // LAT: loads whose row may be past the window read a clamped row instead and the
  // value is discarded where it is used: a load under a branch makes the
  // compiler wait for it inside the branch, one memory round trip each.
  auto load_q = [&](int qt, uint4& a, uint4& b) {
    if constexpr (LAT) {
      const int qi = min(max(qt, 0) * 16 + (lane & 15), p - 1);
      a = *reinterpret_cast<const uint4*>(qb + (size_t)qi * ld + part * 8);
      b = *reinterpret_cast<const uint4*>(qb + (size_t)qi * ld + 32 + part * 8);
    } else {
      const int qi = qt * 16 + (lane & 15);
      a = b = make_uint4(0, 0, 0, 0);
      if (qt >= 0 && qi < p) {
        a = *reinterpret_cast<const uint4*>(qb + (size_t)qi * ld + part * 8);
        b = *reinterpret_cast<const uint4*>(qb + (size_t)qi * ld + 32 + part * 8);
      }
    }
  };

  // Key phase: all of a thread's k / v loads are issued before any is consumed.
  constexpr int NK = MAXKT / 2, NV = (MAXKT + 3) / 4;  // items per 8-lane group at the largest window
  const int d0 = (tid & 7) * 8, g8 = tid >> 3;
  // (LAT: rows past the window load row p - 1; keys and values past it are zeroed where stored)
  uint4 kx[NK], vx[NV][2];
#pragma unroll
  for (int it = 0; it < NK; ++it) {
    const int i = g8 + 32 * it;
    if constexpr (LAT)
      kx[it] = *reinterpret_cast<const uint4*>(qb + E + (size_t)min(i, p - 1) * ld + d0);
    else
      kx[it] = i < p ? *reinterpret_cast<const uint4*>(qb + E + (size_t)i * ld + d0) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int it = 0; it < NV; ++it) {
    const int i = 2 * (g8 + 32 * it);
    const _Float16* src = qb + 2 * E + d0;
    if constexpr (LAT) {
      vx[it][0] = *reinterpret_cast<const uint4*>(src + (size_t)min(i, p - 1) * ld);
      vx[it][1] = *reinterpret_cast<const uint4*>(src + (size_t)min(i + 1, p - 1) * ld);
    } else {
      vx[it][0] = i < p ? *reinterpret_cast<const uint4*>(src + (size_t)i * ld) : make_uint4(0, 0, 0, 0);
      vx[it][1] = i + 1 < p ? *reinterpret_cast<const uint4*>(src + (size_t)(i + 1) * ld) : make_uint4(0, 0, 0, 0);
    }
  }
  // the row's FUTURE flag through the dword holding it: a scalar load, where a
  // byte load would be a vector load waited for to make it uniform (the fut
  // array is a workspace buffer with at least v / 4 bytes of slack after it)
  const uint32_t futw = *reinterpret_cast<const uint32_t*>(d.fut + (r & ~3));
  const bool fut = ((futw >> (8 * (r & 3))) & 0xffu) != 0;
  uint4 qa, qc;
  load_q(tile_at(0), qa, qc);
  // key groups (P32 <= 256: one key a thread), stored after the key phase
  const int kgi = min(tid, p - 1);
  const int kg_at = d.att[row0 + kgi], kg_g = d.grp[row0 + kgi];
  if constexpr (LAT) {
    // the k table rows of key items it + 1 and it + 2 are in flight while item it is rotated
    float ka[3][8], kb[3][8];
    auto load_kt = [&](int it, int buf) {
      const int i = min(g8 + 32 * it, p - 1);
      load_f8(d.rope_k + (size_t)i * 128 + d0, ka[buf]);
      load_f8(d.rope_k + (size_t)i * 128 + 64 + d0, kb[buf]);
    };
    load_kt(0, 0);
    if (NK > 1) load_kt(1, 1);
    // scheduling fences keep the machine scheduler from moving the table loads
    // down to their uses (one round trip per item)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int it = 0; it < NK; ++it) {  // every item (no early exit: the loads stay where issued)
      const int i = g8 + 32 * it;
      if (it + 2 < NK) load_kt(it + 2, (it + 2) % 3);
      __builtin_amdgcn_sched_barrier(0);
      float x[8];
      unpack8(kx[it], x);
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
      ss = lane_sum8(ss);
      // computed for every item (a clamped row past the window) and then zeroed, so the
      // compiler keeps the table loads where they are issued
      half8 o = rotate8(x, ka[it % 3], kb[it % 3], 1.0f / sqrtf(ss / (float)HD + 1e-8f));
      if (i >= p) o = (half8){};
      // (an unconditional store: under a branch the compiler would move the item's
      // table loads into it, after the previous item's wait)
      *reinterpret_cast<uint4*>(Ks + min(i, P16) * LDH + d0) = __builtin_bit_cast(uint4, o);
    }
  } else {
#pragma unroll
    for (int it = 0; it < NK; ++it) {
      const int i = g8 + 32 * it;
      if (i >= P16) break;
      float x[8];
      unpack8(kx[it], x);
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
      ss = lane_sum8(ss);
      half8 o = {};
      if (i < p) {
        float a[8], b[8];
        load_f8(d.rope_k + (size_t)i * 128 + d0, a);
        load_f8(d.rope_k + (size_t)i * 128 + 64 + d0, b);
        o = rotate8(x, a, b, 1.0f / sqrtf(ss / (float)HD + 1e-8f));
      }
      *reinterpret_cast<uint4*>(Ks + i * LDH + d0) = __builtin_bit_cast(uint4, o);
    }
  }
  // A query tile's rows of the q table (norm scale x rotation x xpos scale);
  // the next tile's are loaded after this tile's PV products, so they arrive
  // during the output stores instead of at the head of the tile.
  float ta[16], tb[16];
  auto load_t = [&](int qt2) {
    if constexpr (LAT) {
      const int q2 = min(max(qt2, 0) * 16 + (lane & 15), p - 1);
      const float* t = d.rope_q + (size_t)q2 * 128 + part * 8;
      load_f8(t, ta);
      load_f8(t + 32, ta + 8);
      load_f8(t + 64, tb);
      load_f8(t + 96, tb + 8);
    } else {
      const int q2 = qt2 * 16 + (lane & 15);
      if (qt2 >= 0 && q2 < p) {
        const float* t = d.rope_q + (size_t)q2 * 128 + part * 8;
        load_f8(t, ta);
        load_f8(t + 32, ta + 8);
        load_f8(t + 64, tb);
        load_f8(t + 96, tb + 8);
      }
    }
  };
  if constexpr (LAT) load_t(tile_at(0));  // in flight during the value transposition and the barrier
#pragma unroll
  for (int it = 0; it < NV; ++it) {
    const int i = 2 * (g8 + 32 * it);
    if (i >= P32) break;
    // (selects of values: a select between two named arrays' elements would put
    // them in private memory)
    const half8 hv = __builtin_bit_cast(half8, i < p ? vx[it][0] : make_uint4(0, 0, 0, 0)),
                hw = __builtin_bit_cast(half8, i + 1 < p ? vx[it][1] : make_uint4(0, 0, 0, 0));
    uint32_t* vt2 = reinterpret_cast<uint32_t*>(Vt);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const half2v pr = {hv[e], hw[e]};
      vt2[((d0 + e) * LDV + i) >> 1] = __builtin_bit_cast(uint32_t, pr);
    }
  }
  if (tid < P32) Kg[tid] = tid >= p ? -4 : kg_at ? kg_g : -2;
  __syncthreads();
  if constexpr (!LAT) load_t(tile_at(0));

  _Float16* ost = Os + wave * 16 * LDH;
  for (int k = 0;; ++k) {
    const int qt = tile_at(k);
    if (qt < 0) break;
    const int qi = qt * 16 + (lane & 15);
    uint4 na, nc;  // the next tile's queries, in flight during this tile
    load_q(tile_at(k + 1), na, nc);
    float x[16];
    unpack8(qa, x);
    unpack8(qc, x + 8);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) ss += x[e] * x[e];
    ss = rows_sum(ss);
    half8 bq0 = {}, bq1 = {};
    if (LAT || qi < p) {  // (LAT: rows past the window hold clamped data, never stored)
      const float qinv = 1.0f / sqrtf(ss / (float)HD + 1e-8f);
      bq0 = rotate8(x, ta, tb, qinv);
      bq1 = rotate8(x + 8, ta + 8, tb + 8, qinv);
    }
    qa = na;
    qc = nc;

    // A query without a group (an all-PAD patch) has every key blocked; the
    // reference's softmax then weighs all p keys equally, which a score of 0 on
    // every key < p gives.  Any other query attends at least itself.
    const int kq = Kg[qi];
    const bool blocked = kq < 0;
    const bool need_all = fut || __ballot(qi < p && blocked) != 0;
    const int nkt = need_all ? all_kt : min(all_kt, (qt + 2) & ~1);

    float sc[MAXKT][4];
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < MAXKT; ++kt) {
      if (kt < nkt) {
        floatx4 s = {0.f, 0.f, 0.f, 0.f};
        if (kt * 16 < p) {
          const _Float16* krow = Ks + (kt * 16 + (lane & 15)) * LDH + part * 8;
          s = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const half8*>(krow), bq0, s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const half8*>(krow + 32), bq1, s, 0, 0, 0);
        }
        const int4 kg = *reinterpret_cast<const int4*>(Kg + kt * 16 + part * 4);
        const int kgv[4] = {kg.x, kg.y, kg.z, kg.w};
        const int rel = qi - kt * 16 - part * 4;  // key e of this lane is causal iff e <= rel
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool ok = kgv[e] == kq && (fut || e <= rel);
          sc[kt][e] = blocked ? (kgv[e] != -4 ? 0.0f : -INFINITY) : ok ? s[e] * 0.125f : -INFINITY;
          mx = fmaxf(mx, sc[kt][e]);
        }
      }
    }
    mx = rows_max(mx);
    float sum = 0.0f;
#pragma unroll
    for (int kt = 0; kt < MAXKT; ++kt) {
      if (kt < nkt) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sc[kt][e] = __expf(sc[kt][e] - mx);
          sum += sc[kt][e];
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
          const _Float16* vrow = Vt + (dt * 16 + (lane & 15)) * LDV + 32 * c + part * 4;
          const half4 lo = *reinterpret_cast<const half4*>(vrow);
          const half4 hi = *reinterpret_cast<const half4*>(vrow + 16);
          const half8 bv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, bv, o[dt], 0, 0, 0);
        }
      }
    }
    load_t(tile_at(k + 1));
    // Stage O (16 queries x 64 dims) in the wave's own region, then write
    // 16-byte row chunks.  LDS operations of one wave complete in order; the
    // fences keep the compiler from moving the reads above the writes.
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) ost[(part * 4 + e) * LDH + dt * 16 + (lane & 15)] = (_Float16)o[dt][e];
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
    // the next tile's staging writes must not pass these reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Windows longer than the LDS kernel holds (T0H_LDS_PATCHES): the keys after
// QK-norm + RoPE and the values, transposed, are written once to workspace,
// then every wave streams them for one 16-query tile in 32-key chunks with an
// online softmax (running max and sum per query).
//
// k_time_kprep: one workgroup per (row, head, 32-key chunk).  Layouts (P32 =
// p rounded up to 32; keys >= p zero):
//   kr [row][head][P32][64]  keys, normalized and rotated as k_time_attn does
//   vt [row][head][64][P32]  values by dimension
//   kg [row][P32]            key group if attendable, -2 if not, -4 past p
__global__ __launch_bounds__(256) void k_time_kprep(const AttnDesc d) {
  __shared__ _Float16 vs[32][HD + 8];
  const int p = d.p, P32 = round_up(p, 32), nch = P32 / 32, E = d.E, ld = 3 * E;
  const int ch = blockIdx.x % nch, rh = blockIdx.x / nch, r = rh / d.heads, h = rh % d.heads;
  const int tid = threadIdx.x, kl = tid >> 3, d0 = (tid & 7) * 8, i = ch * 32 + kl;
  const size_t row0 = (size_t)r * p;
  const _Float16* qb = d.qkv + row0 * ld + h * HD;
  uint4 kx = make_uint4(0, 0, 0, 0), vx = make_uint4(0, 0, 0, 0);
  if (i < p) {
    kx = *reinterpret_cast<const uint4*>(qb + E + (size_t)i * ld + d0);
    vx = *reinterpret_cast<const uint4*>(qb + 2 * E + (size_t)i * ld + d0);
  }
  float x[8];
  unpack8(kx, x);
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  ss = lane_sum8(ss);
  half8 o = {};
  if (i < p) {
    float a[8], b[8];
    load_f8(d.rope_k + (size_t)i * 128 + d0, a);
    load_f8(d.rope_k + (size_t)i * 128 + 64 + d0, b);
    o = rotate8(x, a, b, 1.0f / sqrtf(ss / (float)HD + 1e-8f));
  }
  *reinterpret_cast<uint4*>(d.kr + ((size_t)rh * P32 + i) * HD + d0) = __builtin_bit_cast(uint4, o);
  *reinterpret_cast<uint4*>(&vs[kl][d0]) = vx;
  if (h == 0 && tid < 32) {
    const int j = ch * 32 + tid;
    d.kg[(size_t)r * P32 + j] = j >= p ? -4 : d.att[row0 + j] ? d.grp[row0 + j] : -2;
  }
  __syncthreads();
  const int dim = tid >> 2, k8 = (tid & 3) * 8;
  half8 w;
#pragma unroll
  for (int j = 0; j < 8; ++j) w[j] = vs[k8 + j][dim];
  *reinterpret_cast<uint4*>(d.vt + ((size_t)rh * HD + dim) * P32 + ch * 32 + k8) = __builtin_bit_cast(uint4, w);
}

// k_time_attn_long: four waves per workgroup, one 16-query tile each, four
// consecutive tiles of one (row, head) per workgroup (they read the same keys).
// Per 32-key chunk: S^T = K Q^T on two 16-key tiles (lane: query lane%16, keys
// 4(lane/16)..+3 of each tile), the mask, the running max and sum of the
// query's scores, and O^T += V^T P^T, so each lane's output column is its own
// query and the rescale by exp(old max - new max) needs no lane exchange.  The
// next chunk's keys and values are loaded while the current one is computed.
// Mask and blocked-query semantics are k_time_attn's.
__global__ __launch_bounds__(256) void k_time_attn_long(const AttnDesc d) {
  const int p = d.p, P32 = round_up(p, 32), nqt = round_up(p, 16) / 16, quads = (nqt + 3) / 4;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, part = lane >> 4;
  const int rh = blockIdx.x / quads, qt = (blockIdx.x % quads) * 4 + wave;
  if (qt >= nqt) return;  // whole waves; no barrier below
  const int r = rh / d.heads, h = rh % d.heads;
  const int E = d.E, ld = 3 * E;
  const size_t row0 = (size_t)r * p;
  const int qi = qt * 16 + (lane & 15);
  const _Float16* kr = d.kr + (size_t)rh * P32 * HD;
  const _Float16* vt = d.vt + (size_t)rh * HD * P32;
  const int* kgr = d.kg + (size_t)r * P32;

  // the tile's queries, normalized and rotated into the B operand layout
  half8 bq0 = {}, bq1 = {};
  {
    uint4 qa = make_uint4(0, 0, 0, 0), qc = make_uint4(0, 0, 0, 0);
    float ta[16], tb[16];
    if (qi < p) {
      const _Float16* qrow = d.qkv + (row0 + qi) * ld + h * HD;
      qa = *reinterpret_cast<const uint4*>(qrow + part * 8);
      qc = *reinterpret_cast<const uint4*>(qrow + 32 + part * 8);
      const float* t = d.rope_q + (size_t)qi * 128 + part * 8;
      load_f8(t, ta);
      load_f8(t + 32, ta + 8);
      load_f8(t + 64, tb);
      load_f8(t + 96, tb + 8);
    }
    float x[16];
    unpack8(qa, x);
    unpack8(qc, x + 8);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) ss += x[e] * x[e];
    ss = rows_sum(ss);  // the four lanes holding the query (all lanes take part)
    if (qi < p) {
      const float inv = 1.0f / sqrtf(ss / (float)HD + 1e-8f);
      bq0 = rotate8(x, ta, tb, inv);
      bq1 = rotate8(x + 8, ta + 8, tb + 8, inv);
    }
  }
  const int kq = qi < p ? kgr[qi] : -4;
  const bool fut = d.fut[r] != 0, blocked = kq < 0;
  const bool need_all = fut || __ballot(qi < p && blocked) != 0;
  const int nch = need_all ? P32 / 32 : min(P32 / 32, (qt * 16 + 16 + 31) / 32);

  struct Chunk {
    uint4 k[2][2];  // two 16-key tiles x (dims part*8, 32 + part*8)
    uint2 v[4][2];  // per 16-dim tile: keys 4part..+3 and 16 + 4part..+3
    int4 g[2];      // key groups of the lane's keys in each tile
  };
  auto load_chunk = [&](int c, Chunk& ck) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const _Float16* krow = kr + (size_t)(32 * c + 16 * t + (lane & 15)) * HD + part * 8;
      ck.k[t][0] = *reinterpret_cast<const uint4*>(krow);
      ck.k[t][1] = *reinterpret_cast<const uint4*>(krow + 32);
      ck.g[t] = *reinterpret_cast<const int4*>(kgr + 32 * c + 16 * t + part * 4);
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const _Float16* vrow = vt + (size_t)(dt * 16 + (lane & 15)) * P32 + 32 * c + part * 4;
      ck.v[dt][0] = *reinterpret_cast<const uint2*>(vrow);
      ck.v[dt][1] = *reinterpret_cast<const uint2*>(vrow + 16);
    }
  };

  floatx4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = (floatx4){0.f, 0.f, 0.f, 0.f};
  float mrun = -INFINITY, lsum = 0.0f;
  Chunk cur;
  load_chunk(0, cur);
  Chunk nxt = cur;
  for (int c = 0; c < nch; ++c) {
    if (c + 1 < nch) load_chunk(c + 1, nxt);
    float sc[2][4];
    float mc = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      floatx4 s = {0.f, 0.f, 0.f, 0.f};
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, cur.k[t][0]), bq0, s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, cur.k[t][1]), bq1, s, 0, 0, 0);
      const int kgv[4] = {cur.g[t].x, cur.g[t].y, cur.g[t].z, cur.g[t].w};
      const int key0 = 32 * c + 16 * t + part * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = kgv[e] == kq && (fut || key0 + e <= qi);
        sc[t][e] = blocked ? (kgv[e] != -4 ? 0.0f : -INFINITY) : ok ? s[e] * 0.125f : -INFINITY;
        mc = fmaxf(mc, sc[t][e]);
      }
    }
    mc = rows_max(mc);
    const float mnew = fmaxf(mrun, mc);
    const float mref = mnew == -INFINITY ? 0.0f : mnew;  // nothing attended yet: keep zeros
    const float alpha = __expf(mrun - mref);
    mrun = mnew;
    half8 pb;
    float ls = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float w = __expf(sc[t][e] - mref);
        ls += w;
        pb[4 * t + e] = (_Float16)w;
      }
    lsum = lsum * alpha + ls;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
      for (int e = 0; e < 4; ++e) o[dt][e] *= alpha;
      const half4 lo = __builtin_bit_cast(half4, cur.v[dt][0]), hi = __builtin_bit_cast(half4, cur.v[dt][1]);
      const half8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, pb, o[dt], 0, 0, 0);
    }
    cur = nxt;
  }
  const float inv = 1.0f / rows_sum(lsum);
  if (qi < p) {
    _Float16* orow = d.out + (row0 + qi) * E + h * HD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const half4 w = {(_Float16)(o[dt][0] * inv), (_Float16)(o[dt][1] * inv), (_Float16)(o[dt][2] * inv),
                       (_Float16)(o[dt][3] * inv)};
      *reinterpret_cast<half4*>(orow + dt * 16 + part * 4) = w;
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

// Group attention for segments of up to MAXG rows (one row group's variates at
// one patch): the same 8-lane (query row, head) mapping and arithmetic as
// k_group_attn, but with three memory round trips a query whatever the segment
// length: the query row, its group and its segment; the segment's permutation
// entries; every key row's group id and k / v chunks.  Entries past the segment
// read its last row (clamped, no branch: a load under a branch is waited for
// inside it) and are excluded from the softmax, taken over the scores held in
// registers.
template <int MAXG>
__global__ __launch_bounds__(256) void k_group_attn_seg(const AttnDesc d) {
  const int H = d.heads, E = d.E, p = d.p, v = d.v, ld = 3 * E;
  const long long task = ((long long)blockIdx.x * 256 + threadIdx.x) >> 3;
  const int sub = threadIdx.x & 7, d0 = sub * 8;
  if (task >= (long long)v * p * H) return;  // whole 8-lane groups exit together
  const int h = (int)(task % H);
  const long long m = task / H;
  const int r = (int)(m / p), pi = (int)(m % p);
  const _Float16* col = d.qkv + (size_t)h * HD + d0;
  const int gq = d.grp[m];
  const int b = d.seg_begin[r], n = d.seg_len[r];  // n >= 1: a row is in its own segment
  const uint4 qraw = *reinterpret_cast<const uint4*>(col + m * ld);
  float qs[8], kn[8];
  load_f8(d.q_norm + d0, qs);
  load_f8(d.k_norm + d0, kn);
  int jr[MAXG];
#pragma unroll
  for (int i = 0; i < MAXG; ++i) jr[i] = d.perm[b + min(i, n - 1)];
  int kg[MAXG];
  uint4 kr[MAXG], vr[MAXG];
#pragma unroll
  for (int i = 0; i < MAXG; ++i) {
    const long long mk = (long long)jr[i] * p + pi;
    kg[i] = d.grp[mk];
    kr[i] = *reinterpret_cast<const uint4*>(col + mk * ld + E);
    vr[i] = *reinterpret_cast<const uint4*>(col + mk * ld + 2 * E);
  }
  __builtin_amdgcn_sched_barrier(0);  // every member's loads issued before the first is used
  // The segment's softmax is computed for every query (so the loads above stay
  // where they are issued) and replaced for an all-PAD patch below.
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.0f;
  {
    float qn[8];
    unpack8(qraw, qn);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += qn[e] * qn[e];
    const float dq = sqrtf(lane_sum8(ss) / (float)HD + 1e-8f);
#pragma unroll
    for (int e = 0; e < 8; ++e) qn[e] = (qn[e] / dq) * qs[e];
    float sc[MAXG];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < MAXG; ++i) {
      float kx[8];
      unpack8(kr[i], kx);
      float ks = 0.0f, dot = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ks += kx[e] * kx[e];
        dot += qn[e] * (kx[e] * kn[e]);
      }
      ks = lane_sum8(ks);
      dot = lane_sum8(dot);
      sc[i] = i < n && kg[i] == gq ? (dot / sqrtf(ks / (float)HD + 1e-8f)) * 0.125f : -INFINITY;
      mx = fmaxf(mx, sc[i]);
    }
    float l = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXG; ++i) {
      const float pw = i < n && kg[i] == gq ? __expf(sc[i] - mx) : 0.0f;
      float vx[8];
      unpack8(vr[i], vx);
      l += pw;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += pw * vx[e];
    }
    const float inv = 1.0f / l;  // the query's own row is in its segment with its group: l >= 1
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= inv;
  }
  if (gq < 0) {  // all-PAD patch: every score is -1e9, uniform weights over all v rows
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.0f;
    for (int j = 0; j < v; ++j) {
      float vv[8];
      unpack8(*reinterpret_cast<const uint4*>(col + ((long long)j * p + pi) * ld + 2 * E), vv);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += vv[e];
    }
    const float inv = 1.0f / (float)v;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= inv;
  }
  half8 hv;
#pragma unroll
  for (int e = 0; e < 8; ++e) hv[e] = (_Float16)o[e];
  *reinterpret_cast<uint4*>(d.out + m * E + h * HD + d0) = __builtin_bit_cast(uint4, hv);
}

// Group attention by segment: one 8-lane group per (segment, patch, head), each
// lane owning 8 of the 64 dims.  The group loads the q, k and v chunks of every
// member of the segment once and computes every member's query, where
// k_group_attn_seg loads every member's k and v once per query.  The arithmetic of
// a (query, key) pair, and its order, is k_group_attn_seg's, so the results are
// the same.  Three memory round trips a task: the segment's bounds, its
// permutation entries, the members' group ids and chunks (members past the
// segment read its last row and are excluded).
template <int MAXG>
__global__ __launch_bounds__(256) void k_group_attn_sw(const AttnDesc d) {
  const int H = d.heads, E = d.E, p = d.p, v = d.v, ld = 3 * E;
  const long long task = ((long long)blockIdx.x * 256 + threadIdx.x) >> 3;
  const int sub = threadIdx.x & 7, d0 = sub * 8;
  if (task >= (long long)d.n_seg * p * H) return;  // whole 8-lane groups exit together
  const int h = (int)(task % H);
  const long long sp = task / H;
  const int sg = (int)(sp / p), pi = (int)(sp % p);
  const _Float16* col = d.qkv + (size_t)h * HD + d0;
  const int b = d.seg_start[sg];
  const int n = (sg + 1 < d.n_seg ? d.seg_start[sg + 1] : v) - b;  // >= 1
  float qs[8], kn[8];
  load_f8(d.q_norm + d0, qs);
  load_f8(d.k_norm + d0, kn);
  int jr[MAXG];
#pragma unroll
  for (int i = 0; i < MAXG; ++i) jr[i] = d.perm[b + min(i, n - 1)];
  int g[MAXG];
  uint4 qr[MAXG], kr[MAXG], vr[MAXG];
#pragma unroll
  for (int i = 0; i < MAXG; ++i) {
    const long long mk = (long long)jr[i] * p + pi;
    g[i] = d.grp[mk];
    qr[i] = *reinterpret_cast<const uint4*>(col + mk * ld);
    kr[i] = *reinterpret_cast<const uint4*>(col + mk * ld + E);
    vr[i] = *reinterpret_cast<const uint4*>(col + mk * ld + 2 * E);
  }
  __builtin_amdgcn_sched_barrier(0);  // every member's loads issued before the first is used
  // per member key: k * k_norm and its RMS, once for all queries
  float kk[MAXG][8], krs[MAXG];
#pragma unroll
  for (int i = 0; i < MAXG; ++i) {
    float kx[8];
    unpack8(kr[i], kx);
    float ks = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ks += kx[e] * kx[e];
      kk[i][e] = kx[e] * kn[e];
    }
    krs[i] = sqrtf(lane_sum8(ks) / (float)HD + 1e-8f);
  }
#pragma unroll
  for (int a = 0; a < MAXG; ++a) {
    if (a >= n) break;
    const int gq = g[a];
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.0f;
    {
      float qn[8];
      unpack8(qr[a], qn);
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += qn[e] * qn[e];
      const float dq = sqrtf(lane_sum8(ss) / (float)HD + 1e-8f);
#pragma unroll
      for (int e = 0; e < 8; ++e) qn[e] = (qn[e] / dq) * qs[e];
      float sc[MAXG];
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < MAXG; ++i) {
        float dot = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) dot += qn[e] * kk[i][e];
        dot = lane_sum8(dot);
        sc[i] = i < n && g[i] == gq ? (dot / krs[i]) * 0.125f : -INFINITY;
        mx = fmaxf(mx, sc[i]);
      }
      float l = 0.0f;
#pragma unroll
      for (int i = 0; i < MAXG; ++i) {
        const float pw = i < n && g[i] == gq ? __expf(sc[i] - mx) : 0.0f;
        float vx[8];
        unpack8(vr[i], vx);
        l += pw;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += pw * vx[e];
      }
      const float inv = 1.0f / l;  // the query's own row is in its segment with its group: l >= 1
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= inv;
    }
    if (gq < 0) {  // all-PAD patch: every score is -1e9, uniform weights over all v rows
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = 0.0f;
      for (int j = 0; j < v; ++j) {
        float vv[8];
        unpack8(*reinterpret_cast<const uint4*>(col + ((long long)j * p + pi) * ld + 2 * E), vv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += vv[e];
      }
      const float inv = 1.0f / (float)v;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= inv;
    }
    half8 hv;
#pragma unroll
    for (int e = 0; e < 8; ++e) hv[e] = (_Float16)o[e];
    *reinterpret_cast<uint4*>(d.out + ((long long)jr[a] * p + pi) * E + h * HD + d0) = __builtin_bit_cast(uint4, hv);
  }
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(T0H_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

void check_common(const AttnDesc& d) {
  if (!d.qkv || !d.out || !d.grp || !d.q_norm || !d.k_norm) throw Error(T0H_ERR_INVALID_ARG, "attention: null pointer");
  if (d.heads <= 0 || d.E != d.heads * HD)
    throw Error(T0H_ERR_UNSUPPORTED, "attention: head_dim must be 64 (embed_dim = 64 * num_heads)");
}

template <int MAXKT, bool LAT>
void run_time_attn_k(const AttnDesc& d, size_t lds, hipStream_t s) {
  static std::atomic<uint64_t> lds_set{0};  // per instantiation
  allow_dynamic_lds(reinterpret_cast<const void*>(&k_time_attn<MAXKT, LAT>), lds_set);
  hipLaunchKernelGGL((k_time_attn<MAXKT, LAT>), dim3(d.v * d.heads * d.qsplit), dim3(TA_WAVES * 64), lds, s, d);
}
// Latency-bound launches (query tiles split over workgroups: few pairs) take the LAT kernel.
template <int MAXKT>
void run_time_attn(const AttnDesc& d, size_t lds, hipStream_t s) {
  if (d.qsplit > 1)
    run_time_attn_k<MAXKT, true>(d, lds, s);
  else
    run_time_attn_k<MAXKT, false>(d, lds, s);
}

}  // namespace

void launch_time_attention(const AttnDesc& d, hipStream_t s) {
  if (d.v <= 0 || d.p <= 0) return;
  check_common(d);
  if (!d.att || !d.fut || !d.rope_q || !d.rope_k) throw Error(T0H_ERR_INVALID_ARG, "time attention: null pointer");
  if (d.p > T0H_LDS_PATCHES) {
    if (!d.kr || !d.vt || !d.kg) throw Error(T0H_ERR_INVALID_ARG, "time attention: long window without key workspace");
    const int nch = round_up(d.p, 32) / 32, quads = (round_up(d.p, 16) / 16 + 3) / 4;
    hipLaunchKernelGGL(k_time_kprep, dim3(d.v * d.heads * nch), dim3(256), 0, s, d);
    check_hip(hipGetLastError(), "k_time_kprep launch");
    hipLaunchKernelGGL(k_time_attn_long, dim3(d.v * d.heads * quads), dim3(256), 0, s, d);
    check_hip(hipGetLastError(), "k_time_attn_long launch");
    return;
  }
  static_assert(T0H_LDS_PATCHES <= 16 * 16, "the largest instance covers 16 key tiles of 16");
  const size_t lds = time_attn_lds(d.p);
  const int kt = round_up(d.p, 32) / 16;
  // Few (row, head) pairs (one or two series): split each one's query tiles over
  // up to one workgroup per tile so that about a round of the CUs is busy.
  AttnDesc dd = d;
  const int nqt = round_up(d.p, 16) / 16, pairs = d.v * d.heads;
  dd.qsplit = std::max(1, std::min(nqt, 256 / std::max(1, pairs)));
  // (instances close to the window: every key item of an instance is loaded and
  // rotated, rows past the window from a clamped row)
  if (kt <= 4)
    run_time_attn<4>(dd, lds, s);
  else if (kt <= 6)
    run_time_attn<6>(dd, lds, s);
  else if (kt <= 8)
    run_time_attn<8>(dd, lds, s);
  else if (kt <= 10)
    run_time_attn<10>(dd, lds, s);
  else if (kt <= 12)
    run_time_attn<12>(dd, lds, s);
  else
    run_time_attn<16>(dd, lds, s);
  check_hip(hipGetLastError(), "k_time_attn launch");
}

void launch_group_attention(const AttnDesc& d, hipStream_t s) {
  if (d.v <= 0 || d.p <= 0) return;
  check_common(d);
  if (!d.perm || !d.seg_begin || !d.seg_len) throw Error(T0H_ERR_INVALID_ARG, "group attention: null segment arrays");
  const long long lanes = (long long)d.v * d.p * d.heads * 8;
  const dim3 grid((unsigned)((lanes + 255) / 256));
  // by segment when the segment list is there (one task a segment, patch and head)
  const long long seg_lanes = (long long)d.n_seg * d.p * d.heads * 8;
  const dim3 seg_grid((unsigned)((seg_lanes + 255) / 256));
  const bool by_seg = d.seg_start && d.n_seg > 0;
  if (d.seg_max <= 2 && by_seg)
    hipLaunchKernelGGL(k_group_attn_sw<2>, seg_grid, dim3(256), 0, s, d);
  else if (d.seg_max == 3 && by_seg)
    hipLaunchKernelGGL(k_group_attn_sw<3>, seg_grid, dim3(256), 0, s, d);
  else if (d.seg_max <= 4 && by_seg)
    hipLaunchKernelGGL(k_group_attn_sw<4>, seg_grid, dim3(256), 0, s, d);
  else if (d.seg_max <= 8 && by_seg)
    hipLaunchKernelGGL(k_group_attn_sw<8>, seg_grid, dim3(256), 0, s, d);
  else if (d.seg_max <= 4)
    hipLaunchKernelGGL(k_group_attn_seg<4>, grid, dim3(256), 0, s, d);
  else if (d.seg_max <= 8)
    hipLaunchKernelGGL(k_group_attn_seg<8>, grid, dim3(256), 0, s, d);
  else
    hipLaunchKernelGGL(k_group_attn, grid, dim3(256), 0, s, d);
  check_hip(hipGetLastError(), "k_group_attn launch");
}

}  // namespace t0h
