// Quantized-weight GEMM for gfx950 (CDNA4): llama.cpp Q8_0/Q4_0 blocks (and
// f16 rows) are read verbatim from HBM and dequantized inside the kernel.
//
// Two kernels implement the t0-fast `linear()` contract (crates/t0-fast/src/
// model.rs:406-504; ops.rs:40-42, y = x W^T + b):
//
//  * k_gemm — MFMA tile kernel for large M.  256x128 (M > 128) or 128x128 output
//    tile per workgroup of 8 or 4 waves, 64x64 each, v_mfma_f32_16x16x32_f16.  Per 64-wide K
//    step each thread fetches one 32-value weight block (34 B Q8_0 / 18 B Q4_0 /
//    64 B f16) and one 32-value activation strip into registers while the
//    previous step's MFMAs run, then dequantizes the block to f16 with packed
//    f16 math (exact integer-to-f16 via the 0x6400 exponent trick, then one
//    rounding of d*q) into a double-buffered LDS tile.  Accumulation is f32.
//    Fused epilogues: bias, ReLU, f16/f32 store, residual add into the f32
//    stream, SwiGLU (gate column j paired with up column H+j in one tile), and a
//    row-gathered table add (type embeddings).  Workgroups are remapped so that
//    each XCD walks a contiguous range of tiles (A strips and weights stay in
//    that XCD's L2).
//
//  * k_gemv — bandwidth kernel for small M (<= 2 rows per pass).  Each
//    workgroup stages 16 contiguous weight rows into LDS with 16-byte coalesced
//    loads and computes them in exact f32 (f32(d)*q dequant, f32 activations,
//    f32 accumulation), reducing across the workgroup with a reduce-scatter
//    shuffle tree.
//
// Dequantization math is the reference's (gguf.rs:116-126, 159-174): Q8_0
// value = f32(d) * i8, Q4_0 value = f32(d) * (nibble - 8); low nibble of byte j
// is value j, high nibble value j+16.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "kernels.h"
#include "t0hip_internal.h"

namespace t0h {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int TN = 128, TK = 64, LDK = TK + 8;

__host__ __device__ constexpr int block_bytes(int wt) { return wt == T0H_Q8_0 ? 34 : (wt == T0H_Q4_0 ? 18 : 0); }

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// 4 signed int8 (one dword) -> 4 f16 values d*q as 2 dwords.  (1024+u) - 1152 is
// exact in f16, and the packed multiply rounds the exact product d*q once.
__device__ __forceinline__ void q8x4_f16(uint32_t w, half2v dd, uint32_t& o0, uint32_t& o1) {
  const uint32_t u = w ^ 0x80808080u;
  const half2v off = {(_Float16)1152.0f, (_Float16)1152.0f};
  half2v h0 = __builtin_bit_cast(half2v, perm(0x64646464u, u, 0x04010400u)) - off;
  half2v h1 = __builtin_bit_cast(half2v, perm(0x64646464u, u, 0x04030402u)) - off;
  o0 = __builtin_bit_cast(uint32_t, h0 * dd);
  o1 = __builtin_bit_cast(uint32_t, h1 * dd);
}
// 4 nibbles (one per byte, values 0..15) -> 4 f16 values d*(n-8).
__device__ __forceinline__ void q4x4_f16(uint32_t nib, half2v dd, uint32_t& o0, uint32_t& o1) {
  const half2v off = {(_Float16)1032.0f, (_Float16)1032.0f};
  half2v h0 = __builtin_bit_cast(half2v, perm(0x64646464u, nib, 0x04010400u)) - off;
  half2v h1 = __builtin_bit_cast(half2v, perm(0x64646464u, nib, 0x04030402u)) - off;
  o0 = __builtin_bit_cast(uint32_t, h0 * dd);
  o1 = __builtin_bit_cast(uint32_t, h1 * dd);
}

// silu_mul.wgsl:21 g/(1+exp(-g)); reciprocal via v_rcp_f32 (output is rounded to f16).
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// ---------------------------------------------------------------------------
// MFMA tile kernel.  NWM waves along M x 2 along N, each wave 64x64; tile
// (64*NWM) x 128 x 64.  Loader roles: A strip = 32 activations per thread (row
// tid/2, half tid%2); weights = 64/NWM values per thread.
// ---------------------------------------------------------------------------
template <int NWM>
struct TileCfg {
  static constexpr int BM = 64 * NWM, NT = 128 * NWM, BV = 64 / NWM;
  static constexpr int LDS = 2 * (BM + TN) * LDK * 2;
};

// Loads the raw weight bytes of one thread's share of a K step.
// BV == 32: one whole 32-value block (row tid/2, block tid%2).
// BV == 16: Q8_0 / f16: half a block (16 consecutive values); Q4_0: 8 quant
// bytes = values {8h..8h+7} and {16+8h..16+8h+7} of the block.
template <int WT, bool AL4, int BV>
__device__ __forceinline__ void load_w(const uint8_t* wrow, int kt, int part, uint32_t (&br)[16]) {
  if (WT == T0H_F16) {
    const uint4* src = reinterpret_cast<const uint4*>(wrow + (size_t)(kt * TK + part * BV) * 2);
#pragma unroll
    for (int i = 0; i < BV / 8; ++i) {
      const uint4 v = src[i];
      br[4 * i + 0] = v.x;
      br[4 * i + 1] = v.y;
      br[4 * i + 2] = v.z;
      br[4 * i + 3] = v.w;
    }
    return;
  }
  constexpr int BB = block_bytes(WT);
  if (BV == 32) {
    const int lh = part;
    if (AL4) {
      const uint32_t* src = reinterpret_cast<const uint32_t*>(wrow) + (WT == T0H_Q8_0 ? 17 * kt + 8 * lh : 9 * kt + 4 * lh);
      constexpr int NW = WT == T0H_Q8_0 ? 9 : 5;
#pragma unroll
      for (int i = 0; i < NW; ++i) br[i] = src[i];
    } else {
      const uint16_t* src = reinterpret_cast<const uint16_t*>(wrow + (size_t)(2 * kt + lh) * BB);
      constexpr int NQ = WT == T0H_Q8_0 ? 8 : 4;
      br[0] = src[0];
#pragma unroll
      for (int i = 0; i < NQ; ++i) br[1 + i] = (uint32_t)src[1 + 2 * i] | ((uint32_t)src[2 + 2 * i] << 16);
    }
    return;
  }
  // BV == 16: br[0] = scale dword, br[1..] = quant dwords (funnel-shifted in decode)
  const int b = part >> 1, h = part & 1;
  if (AL4) {
    const uint32_t* base = reinterpret_cast<const uint32_t*>(wrow) + (WT == T0H_Q8_0 ? 17 * kt : 9 * kt);
    if (WT == T0H_Q8_0) {
      br[0] = base[b ? 8 : 0];
      const uint32_t* q = base + (b ? 8 + 4 * h : 4 * h);
#pragma unroll
      for (int i = 0; i < 5; ++i) br[1 + i] = q[i];
    } else {
      br[0] = base[b ? 4 : 0];
      const uint32_t* q = base + (b ? 4 + 2 * h : 2 * h);
#pragma unroll
      for (int i = 0; i < 3; ++i) br[1 + i] = q[i];
    }
  } else {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(wrow + (size_t)(2 * kt + b) * BB);
    br[0] = src[0];
    constexpr int NQ = WT == T0H_Q8_0 ? 4 : 2;  // dwords of quants
    const uint16_t* q = src + 1 + (WT == T0H_Q8_0 ? 8 * h : 4 * h);
#pragma unroll
    for (int i = 0; i < NQ; ++i) br[1 + i] = (uint32_t)q[2 * i] | ((uint32_t)q[2 * i + 1] << 16);
  }
}

// Dequantizes a thread's share to packed f16 (out[] in k order; for Q4_0 with
// BV == 16, out[0..3] are the low-nibble values and out[4..7] the high ones).
template <int WT, bool AL4, int BV>
__device__ __forceinline__ void dequant_w(const uint32_t (&br)[16], int part, uint32_t (&out)[16]) {
  if (WT == T0H_F16) {
#pragma unroll
    for (int i = 0; i < BV / 2; ++i) out[i] = br[i];
    return;
  }
  uint32_t dbits, q[8];
  constexpr int NQ = BV == 32 ? (WT == T0H_Q8_0 ? 8 : 4) : (WT == T0H_Q8_0 ? 4 : 2);
  if (BV == 32) {
    const int lh = part;
    if (AL4) {
      const uint32_t sel = lh ? 0x07060504u : 0x05040302u;
      dbits = lh ? (br[0] >> 16) : (br[0] & 0xffffu);
#pragma unroll
      for (int i = 0; i < NQ; ++i) q[i] = perm(br[i + 1], br[i], sel);
    } else {
      dbits = br[0] & 0xffffu;
#pragma unroll
      for (int i = 0; i < NQ; ++i) q[i] = br[1 + i];
    }
  } else {
    const int b = part >> 1;
    if (AL4) {
      dbits = b ? (br[0] >> 16) : (br[0] & 0xffffu);
      const uint32_t sel = b ? 0x07060504u : 0x05040302u;
#pragma unroll
      for (int i = 0; i < NQ; ++i) q[i] = perm(br[i + 2], br[i + 1], sel);
    } else {
      dbits = br[0] & 0xffffu;
#pragma unroll
      for (int i = 0; i < NQ; ++i) q[i] = br[1 + i];
    }
  }
  const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)dbits);
  const half2v dd = {dh, dh};
  if (WT == T0H_Q8_0) {
#pragma unroll
    for (int i = 0; i < NQ; ++i) q8x4_f16(q[i], dd, out[2 * i], out[2 * i + 1]);
  } else {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      q4x4_f16(q[i] & 0x0f0f0f0fu, dd, out[2 * i], out[2 * i + 1]);
      q4x4_f16((q[i] >> 4) & 0x0f0f0f0fu, dd, out[2 * NQ + 2 * i], out[2 * NQ + 2 * i + 1]);
    }
  }
}

template <int WT, bool A32, int EPI, bool AL4, int NWM>
__global__ __launch_bounds__(128 * NWM) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm(const GemmDesc d) {
  using C = TileCfg<NWM>;
  constexpr int BM = C::BM, BV = C::BV;
  extern __shared__ __align__(16) _Float16 smem[];
  _Float16* As = smem;                 // [2][BM][LDK]
  _Float16* Bs = smem + 2 * BM * LDK;  // [2][TN][LDK]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int M = d.M, N = d.N, K = d.K;
  const int tiles_n = EPI == EPI_SWIGLU_F16 ? (N + 63) / 64 : (N + TN - 1) / TN;

  // XCD-aware remap: blocks are dispatched round-robin over 8 XCDs; give each
  // XCD a contiguous range of logical tiles (N fastest within an M strip).
  const int total = gridDim.x, bid = blockIdx.x;
  const int per = total / 8;
  const int logical = bid < per * 8 ? (bid % 8) * per + bid / 8 : bid;
  const int tm = logical / tiles_n, tn = logical % tiles_n;
  const int m0 = tm * BM;

  // A loader: row ar, half ah (32 values); rows past M read row M-1
  const int ar = tid >> 1, ah = tid & 1;
  const int amc = min(m0 + ar, M - 1);
  // weight loader: tile row brow, part bp; rows past N read row 0
  constexpr int PARTS = 64 / BV;
  const int brow = tid / PARTS, bp = tid % PARTS;
  const int bp_lo = bp & (PARTS / 2 - 1);  // the same share of the step's first block
  int wrow;
  bool bvalid;
  if (EPI == EPI_SWIGLU_F16) {
    const int g = tn * 64 + (brow & 63);
    bvalid = g < N;
    wrow = brow < 64 ? g : N + g;  // gate rows then up rows (weight has 2N rows)
  } else {
    wrow = tn * TN + brow;
    bvalid = wrow < N;
  }
  const size_t rowb = WT == T0H_F16 ? (size_t)K * 2 : (size_t)(K / 32) * block_bytes(WT);
  const uint8_t* wbase = static_cast<const uint8_t*>(d.w) + (size_t)(bvalid ? wrow : 0) * rowb;
  // k offset (in values) of this thread's weight share inside a K step
  const int bk0 = BV == 32 ? bp * 32 : (WT == T0H_Q4_0 ? (bp >> 1) * 32 + (bp & 1) * 8 : bp * 16);

  // Raw global data of one K step held in registers between its load and its
  // LDS store.  Two stages are in flight: the loads for step kt+2 are issued
  // while step kt is multiplied, so a fresh activation strip (which every
  // workgroup of an XCD requests at the same time) has two steps of MFMA work
  // to arrive from HBM.
  struct Stage {
    uint32_t a[A32 ? 32 : 16];
    uint32_t b[16];
  };

  // Branch-free loads: rows past M or N read a clamped valid row (their
  // outputs are never stored); only the K tail of the last step (K % 64 == 32)
  // is zeroed, under a uniform branch, so the stage stays in registers.
  auto load_global = [&](Stage& st, int kt) {
    const int k0 = kt * TK + ah * 32;
    const int k0c = k0 < K ? k0 : k0 - 32;
    if (A32) {
      const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(d.a) + (size_t)amc * d.lda + k0c);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float4 v = src[i];
        st.a[4 * i + 0] = __builtin_bit_cast(uint32_t, v.x);
        st.a[4 * i + 1] = __builtin_bit_cast(uint32_t, v.y);
        st.a[4 * i + 2] = __builtin_bit_cast(uint32_t, v.z);
        st.a[4 * i + 3] = __builtin_bit_cast(uint32_t, v.w);
      }
    } else {
      const uint4* src = reinterpret_cast<const uint4*>(static_cast<const _Float16*>(d.a) + (size_t)amc * d.lda + k0c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint4 v = src[i];
        st.a[4 * i + 0] = v.x;
        st.a[4 * i + 1] = v.y;
        st.a[4 * i + 2] = v.z;
        st.a[4 * i + 3] = v.w;
      }
    }
    load_w<WT, AL4, BV>(wbase, kt, kt * TK + bk0 < K ? bp : bp_lo, st.b);
  };

  auto store_lds = [&](Stage& st, int buf, int kt) {
    if (kt * TK + TK > K) {  // uniform: the last step of a K % 64 == 32 problem
      const bool aok = kt * TK + ah * 32 < K;
#pragma unroll
      for (int i = 0; i < (A32 ? 32 : 16); ++i) st.a[i] = aok ? st.a[i] : 0u;
    }
    uint32_t out[16];
    if (A32) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        half2v h = {(_Float16)__builtin_bit_cast(float, st.a[2 * i]), (_Float16)__builtin_bit_cast(float, st.a[2 * i + 1])};
        out[i] = __builtin_bit_cast(uint32_t, h);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) out[i] = st.a[i];
    }
    uint4* adst = reinterpret_cast<uint4*>(As + (size_t)buf * BM * LDK + ar * LDK + ah * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) adst[i] = make_uint4(out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]);
    const bool bok = kt * TK + bk0 < K;
    uint32_t wq[16];
    dequant_w<WT, AL4, BV>(st.b, bok ? bp : bp_lo, wq);
    if (kt * TK + TK > K) {
#pragma unroll
      for (int i = 0; i < BV / 2; ++i) wq[i] = bok ? wq[i] : 0u;
    }
    _Float16* brow_p = Bs + (size_t)buf * TN * LDK + brow * LDK;
    if (BV == 16 && WT == T0H_Q4_0) {
      *reinterpret_cast<uint4*>(brow_p + bk0) = make_uint4(wq[0], wq[1], wq[2], wq[3]);
      *reinterpret_cast<uint4*>(brow_p + bk0 + 16) = make_uint4(wq[4], wq[5], wq[6], wq[7]);
    } else {
#pragma unroll
      for (int i = 0; i < BV / 8; ++i)
        reinterpret_cast<uint4*>(brow_p + bk0)[i] = make_uint4(wq[4 * i], wq[4 * i + 1], wq[4 * i + 2], wq[4 * i + 3]);
    }
  };

  // Each wave owns a 64x64 block as 2x2 tiles of v_mfma_f32_32x32x16_f16
  // (measured on MI355X: this shape sustains ~2.2 PFLOP/s even at one wave per
  // SIMD, where 16x16x32 needs 16+ independent chains and several waves).
  // Operand lane layout: lane l holds row (A) / column (B) l%32 and k-slots
  // (l/32)*8 .. +8 of the 16-wide K slice.
  // B-tile rows of the wave's two column tiles; SwiGLU pairs gate tile j=0 with
  // the up tile j=1 holding the same hidden columns.
  int bcol[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    bcol[j] = EPI == EPI_SWIGLU_F16 ? j * 64 + wn * 32 : wn * 64 + j * 32;

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  auto compute = [&](int buf) {
    const _Float16* At = As + (size_t)buf * BM * LDK + (wm * 64 + (lane & 31)) * LDK + (lane >> 5) * 8;
    const _Float16* Bt = Bs + (size_t)buf * TN * LDK + (lane & 31) * LDK + (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < TK / 16; ++kk) {
      half8 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const half8*>(At + i * 32 * LDK + kk * 16);
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = *reinterpret_cast<const half8*>(Bt + bcol[j] * LDK + kk * 16);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  // Steps alternate between (LDS buffer 0, stage s0) and (buffer 1, stage s1);
  // the loop body covers two steps so the stage registers are indexed statically.
  const int KT = (K + TK - 1) / TK;
  Stage s0, s1;
  load_global(s0, 0);
  if (KT > 1) load_global(s1, 1);
  store_lds(s0, 0, 0);
  __syncthreads();
  for (int kt = 0; kt < KT; kt += 2) {
    if (kt + 2 < KT) load_global(s0, kt + 2);
    compute(0);
    if (kt + 1 < KT) store_lds(s1, 1, kt + 1);
    __syncthreads();
    if (kt + 1 >= KT) break;
    if (kt + 3 < KT) load_global(s1, kt + 3);
    compute(1);
    if (kt + 2 < KT) store_lds(s0, 0, kt + 2);
    __syncthreads();
  }

  // Epilogue, staged through LDS (free after the main loop's last barrier):
  // each wave writes a 32-row slice of its results (bias, SwiGLU applied) as
  // f32 into its own LDS region, then streams the slice out in 16-byte row
  // chunks (coalesced f32/f16 stores, vector residual read-modify-write).
  // In each 32x32 MFMA tile lane l holds column l%32, rows (e/4)*8 + (l/32)*4 + e%4.
  constexpr int W = EPI == EPI_SWIGLU_F16 ? 32 : 64;  // output columns per wave
  constexpr int SLD = W + 4;                          // staging row stride (floats)
  float* stage = reinterpret_cast<float*>(smem) + wave * 32 * SLD;
  const int cbase = EPI == EPI_SWIGLU_F16 ? tn * 64 + wn * 32 : tn * TN + wn * 64;  // first output column
  const int lc = lane & 31, lr = (lane >> 5) * 4;
  float bj[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = EPI == EPI_SWIGLU_F16 ? cbase + lc + (j ? N : 0) : cbase + j * 32 + lc;
    bj[j] = (d.bias && (EPI == EPI_SWIGLU_F16 ? cbase + lc < N : col < N)) ? d.bias[col] : 0.0f;
  }
  const bool vec_ok = (d.ldy & 3) == 0 && (N & 3) == 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int r = (e >> 2) * 8 + lr + (e & 3);
      if (EPI == EPI_SWIGLU_F16) {
        stage[r * SLD + lc] = silu(acc[i][0][e] + bj[0]) * (acc[i][1][e] + bj[1]);
      } else {
        stage[r * SLD + lc] = acc[i][0][e] + bj[0];
        stage[r * SLD + 32 + lc] = acc[i][1][e] + bj[1];
      }
    }
    __syncthreads();
    const int row0 = m0 + wm * 64 + i * 32;
#pragma unroll
    for (int t = 0; t < 32 * W / 4 / 64; ++t) {
      const int idx = t * 64 + lane;
      const int r = idx / (W / 4), c = (idx % (W / 4)) * 4;
      const int row = row0 + r, col = cbase + c;
      if (row >= M || col >= N) continue;
      float4 v = *reinterpret_cast<const float4*>(stage + r * SLD + c);
      const size_t o = (size_t)row * d.ldy + col;
      if (vec_ok) {
        if (EPI == EPI_STORE_F32 && d.row_add) {
          const float4 t4 = *reinterpret_cast<const float4*>(d.row_add + (size_t)d.row_add_idx[row] * N + col);
          v.x += t4.x; v.y += t4.y; v.z += t4.z; v.w += t4.w;
        }
        if (EPI != EPI_RESID_F32 && d.relu) {
          v.x = fmaxf(v.x, 0.0f); v.y = fmaxf(v.y, 0.0f); v.z = fmaxf(v.z, 0.0f); v.w = fmaxf(v.w, 0.0f);
        }
        if (EPI == EPI_RESID_F32) {
          float4* y = reinterpret_cast<float4*>(static_cast<float*>(d.y) + o);
          const float4 old = *y;
          *y = make_float4(old.x + v.x, old.y + v.y, old.z + v.z, old.w + v.w);
        } else if (EPI == EPI_STORE_F32) {
          *reinterpret_cast<float4*>(static_cast<float*>(d.y) + o) = v;
        } else {
          half4 h = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
          *reinterpret_cast<half4*>(static_cast<_Float16*>(d.y) + o) = h;
        }
      } else {
        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (col + q >= N) break;
          float x = vv[q];
          if (EPI == EPI_STORE_F32 && d.row_add) x += d.row_add[(size_t)d.row_add_idx[row] * N + col + q];
          if (EPI != EPI_RESID_F32 && d.relu) x = fmaxf(x, 0.0f);
          if (EPI == EPI_RESID_F32) {
            float* y = static_cast<float*>(d.y) + o + q;
            *y = *y + x;
          } else if (EPI == EPI_STORE_F32) {
            static_cast<float*>(d.y)[o + q] = x;
          } else {
            static_cast<_Float16*>(d.y)[o + q] = (_Float16)x;
          }
        }
      }
    }
    if (i == 0) __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Small-M kernel: 16 weight rows per workgroup staged in LDS, exact f32 math.
// ---------------------------------------------------------------------------
constexpr int GV_NR = 16;

template <int WT>
__device__ __forceinline__ void dequant8_lds(const uint8_t* row, int c, float (&w)[8]) {
  if (WT == T0H_F16) {
    const uint4 v = *reinterpret_cast<const uint4*>(row + (size_t)c * 16);
    const half8 h = __builtin_bit_cast(half8, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = (float)h[e];
  } else {
    const int blk = c >> 2, sub = c & 3;
    const uint8_t* b = row + (size_t)blk * block_bytes(WT);
    const uint16_t* b16 = reinterpret_cast<const uint16_t*>(b);
    const float dv = (float)__builtin_bit_cast(_Float16, b16[0]);
    if (WT == T0H_Q8_0) {
      const uint16_t* q = b16 + 1 + sub * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t u = q[i];
        w[2 * i] = dv * (float)(int8_t)(u & 0xff);
        w[2 * i + 1] = dv * (float)(int8_t)(u >> 8);
      }
    } else {
      const uint16_t* q = b16 + 1 + (sub & 1) * 4;
      const int sh = sub < 2 ? 0 : 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t u = q[i];
        w[2 * i] = dv * ((float)((u >> sh) & 0xf) - 8.0f);
        w[2 * i + 1] = dv * ((float)((u >> (8 + sh)) & 0xf) - 8.0f);
      }
    }
  }
}

template <int V>
__device__ __forceinline__ float wave_reduce_scatter(float (&v)[V], int lane, int& idx) {
  idx = 0;
  int mask = 32;
#pragma unroll
  for (int half = V / 2; half >= 1; half /= 2) {
    const bool up = (lane & mask) != 0;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float send = up ? v[i] : v[i + half];
      const float keep = up ? v[i + half] : v[i];
      v[i] = keep + __shfl_xor(send, mask);
    }
    if (up) idx += half;
    mask >>= 1;
  }
  for (; mask >= 1; mask >>= 1) v[0] += __shfl_xor(v[0], mask);
  return v[0];
}

template <int WT, bool A32, int EPI, int MT>
__global__ __launch_bounds__(256) void k_gemv(const GemmDesc d) {
  extern __shared__ __align__(16) uint8_t sm[];
  constexpr int V = GV_NR * MT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int M = d.M, N = d.N, K = d.K;
  const size_t rb = WT == T0H_F16 ? (size_t)K * 2 : (size_t)(K / 32) * block_bytes(WT);
  const uint8_t* W = static_cast<const uint8_t*>(d.w);
  const int m0 = blockIdx.y * MT;

  // stage rows (two 8-row segments for SwiGLU: gate rows g0.., up rows N+g0..)
  const int nseg = EPI == EPI_SWIGLU_F16 ? 2 : 1;
  const int seg_rows = GV_NR / nseg;
  const int r0 = blockIdx.x * seg_rows;
  const int valid = min(seg_rows, N - r0);
  for (int sgi = 0; sgi < nseg; ++sgi) {
    const size_t src_row = (size_t)(sgi == 0 ? r0 : N + r0);
    const uint8_t* src = W + src_row * rb;
    uint8_t* dst = sm + (size_t)sgi * seg_rows * rb;
    const size_t bytes = (size_t)valid * rb;
    const size_t n16 = bytes / 16;
    for (size_t i = tid; i < n16; i += 256)
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
    for (size_t i = n16 * 16 + tid; i < bytes; i += 256) dst[i] = src[i];
  }
  __syncthreads();

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.0f;
  for (int c = tid; c < K / 8; c += 256) {
    float xv[MT][8];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m0 + mt;
      if (m < M) {
        if (A32) {
          const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(d.a) + (size_t)m * d.lda + c * 8);
          const float4 a = src[0], b = src[1];
          xv[mt][0] = a.x; xv[mt][1] = a.y; xv[mt][2] = a.z; xv[mt][3] = a.w;
          xv[mt][4] = b.x; xv[mt][5] = b.y; xv[mt][6] = b.z; xv[mt][7] = b.w;
        } else {
          const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const _Float16*>(d.a) + (size_t)m * d.lda + c * 8);
          const half8 h = __builtin_bit_cast(half8, u);
#pragma unroll
          for (int e = 0; e < 8; ++e) xv[mt][e] = (float)h[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[mt][e] = 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < GV_NR; ++r) {
      float w[8];
      dequant8_lds<WT>(sm + (size_t)r * rb, c, w);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r * MT + mt] = fmaf(w[e], xv[mt][e], acc[r * MT + mt]);
    }
  }
  int idx;
  const float part = wave_reduce_scatter<V>(acc, lane, idx);
  __syncthreads();  // staged rows no longer needed: reuse LDS for the reduction
  float* red = reinterpret_cast<float*>(sm);
  constexpr int LOWMASK = 64 / V - 1;
  if ((lane & LOWMASK) == 0) red[wave * V + idx] = part;
  __syncthreads();
  float* fin = red + 4 * V;
  if (tid < V) fin[tid] = red[tid] + red[V + tid] + red[2 * V + tid] + red[3 * V + tid];
  __syncthreads();
  if (EPI == EPI_SWIGLU_F16) {
    if (tid < V / 2) {
      const int r = tid / MT, mt = tid % MT;
      const int g = r0 + r, m = m0 + mt;
      if (r < valid && m < M) {
        const float gate = fin[tid] + (d.bias ? d.bias[g] : 0.0f);
        const float up = fin[tid + V / 2] + (d.bias ? d.bias[N + g] : 0.0f);
        static_cast<_Float16*>(d.y)[(size_t)m * d.ldy + g] = (_Float16)(silu(gate) * up);
      }
    }
  } else if (tid < V) {
    const int r = tid / MT, mt = tid % MT;
    const int n = r0 + r, m = m0 + mt;
    if (r < valid && m < M) {
      float v = fin[tid] + (d.bias ? d.bias[n] : 0.0f);
      const size_t o = (size_t)m * d.ldy + n;
      if (EPI == EPI_RESID_F32) {
        float* y = static_cast<float*>(d.y);
        y[o] = y[o] + v;
      } else {
        if (EPI == EPI_STORE_F32 && d.row_add) v = v + d.row_add[(size_t)d.row_add_idx[m] * N + n];
        if (d.relu) v = v > 0.0f ? v : 0.0f;
        if (EPI == EPI_STORE_F32)
          static_cast<float*>(d.y)[o] = v;
        else
          static_cast<_Float16*>(d.y)[o] = (_Float16)v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Bit-exact dequantization to f32 (gguf.rs:213-226)
// ---------------------------------------------------------------------------
template <int WT>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* w, size_t n, float* out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (WT == T0H_F32) {
    if (i < n) out[i] = reinterpret_cast<const float*>(w)[i];
  } else if (WT == T0H_F16) {
    if (i < n) out[i] = (float)reinterpret_cast<const _Float16*>(w)[i];
  } else {
    if (i >= n / 32) return;
    const uint16_t* b = reinterpret_cast<const uint16_t*>(w + i * block_bytes(WT));
    const float dv = (float)__builtin_bit_cast(_Float16, b[0]);
    float* o = out + i * 32;
    if (WT == T0H_Q8_0) {
      for (int j = 0; j < 16; ++j) {
        const uint32_t u = b[1 + j];
        o[2 * j] = dv * (float)(int8_t)(u & 0xff);
        o[2 * j + 1] = dv * (float)(int8_t)(u >> 8);
      }
    } else {
      for (int j = 0; j < 8; ++j) {
        const uint32_t u = b[1 + j];
        o[2 * j] = dv * ((float)(u & 0xf) - 8.0f);
        o[2 * j + 16] = dv * ((float)((u >> 4) & 0xf) - 8.0f);
        o[2 * j + 1] = dv * ((float)((u >> 8) & 0xf) - 8.0f);
        o[2 * j + 17] = dv * ((float)((u >> 12) & 0xf) - 8.0f);
      }
    }
  }
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(T0H_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

template <int WT, bool A32, int EPI, bool AL4, int NWM>
void run_gemm(const GemmDesc& d, hipStream_t s) {
  using C = TileCfg<NWM>;
  const int tiles_n = EPI == EPI_SWIGLU_F16 ? (d.N + 63) / 64 : (d.N + TN - 1) / TN;
  const int tiles_m = (d.M + C::BM - 1) / C::BM;
  static bool attr_set = false;  // per instantiation
  if (!attr_set) {
    check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm<WT, A32, EPI, AL4, NWM>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS),
              "hipFuncSetAttribute(k_gemm)");
    attr_set = true;
  }
  hipLaunchKernelGGL((k_gemm<WT, A32, EPI, AL4, NWM>), dim3(tiles_m * tiles_n), dim3(C::NT), C::LDS, s, d);
  check_hip(hipGetLastError(), "k_gemm launch");
}

// 256-row tiles halve the dequant work per MFMA but hold one workgroup per CU,
// so the workgroups run in lock-step; measured faster only for the f16-store
// (QKV) shape at config-4 scale.
template <int WT, bool A32, int EPI, bool AL4>
void run_gemm_m(const GemmDesc& d, hipStream_t s) {
  if (EPI == EPI_STORE_F16 && d.M > 4096)
    run_gemm<WT, A32, EPI, AL4, 4>(d, s);
  else
    run_gemm<WT, A32, EPI, AL4, 2>(d, s);
}

template <int WT, bool A32, int EPI, int MT>
void run_gemv(const GemmDesc& d, hipStream_t s) {
  const size_t rb = WT == T0H_F16 ? (size_t)d.K * 2 : (size_t)(d.K / 32) * block_bytes(WT);
  const size_t lds = std::max<size_t>(GV_NR * rb, 5 * GV_NR * MT * sizeof(float));
  const int seg_rows = EPI == EPI_SWIGLU_F16 ? GV_NR / 2 : GV_NR;
  const int gx = (d.N + seg_rows - 1) / seg_rows, gy = (d.M + MT - 1) / MT;
  if (lds > 160 * 1024) throw Error(T0H_ERR_UNSUPPORTED, "gemv: K too large for the LDS row stage");
  check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv<WT, A32, EPI, MT>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
            "hipFuncSetAttribute(k_gemv)");
  hipLaunchKernelGGL((k_gemv<WT, A32, EPI, MT>), dim3(gx, gy), dim3(256), lds, s, d);
  check_hip(hipGetLastError(), "k_gemv launch");
}

template <int WT, bool A32, int EPI>
void dispatch_gemv(const GemmDesc& d, hipStream_t s) {
  if (d.M == 1)
    run_gemv<WT, A32, EPI, 1>(d, s);
  else
    run_gemv<WT, A32, EPI, 2>(d, s);
}

template <int WT, bool A32, int EPI>
void dispatch_w(const GemmDesc& d, int force, hipStream_t s) {
  const bool mfma = force == 1 || (force == 0 && d.M > 16);
  if (mfma) {
    if (WT != T0H_F16 && d.K % 64 == 0)
      run_gemm_m<WT, A32, EPI, true>(d, s);
    else
      run_gemm_m<WT, A32, EPI, false>(d, s);
  } else {
    dispatch_gemv<WT, A32, EPI>(d, s);
  }
}

template <bool A32, int EPI>
void dispatch_type(const GemmDesc& d, int force, hipStream_t s) {
  switch (d.wtype) {
    case T0H_F16: dispatch_w<T0H_F16, A32, EPI>(d, force, s); return;
    case T0H_Q8_0: dispatch_w<T0H_Q8_0, A32, EPI>(d, force, s); return;
    case T0H_Q4_0: dispatch_w<T0H_Q4_0, A32, EPI>(d, force, s); return;
  }
  throw Error(T0H_ERR_UNSUPPORTED, "gemm: weight type must be F16, Q8_0 or Q4_0");
}

}  // namespace

void launch_gemm_forced(const GemmDesc& d, int force, hipStream_t s) {
  if (d.M <= 0 || d.N <= 0) return;
  if (!d.w || !d.a || !d.y) throw Error(T0H_ERR_INVALID_ARG, "gemm: null pointer");
  if (d.K <= 0 || d.K % 32) throw Error(T0H_ERR_UNSUPPORTED, "gemm: K must be a positive multiple of 32");
  if (d.lda < d.K || d.lda % 8) throw Error(T0H_ERR_INVALID_ARG, "gemm: lda must be >= K and a multiple of 8");
  const int ncols = d.N;
  if (d.ldy < ncols) throw Error(T0H_ERR_INVALID_ARG, "gemm: ldy < N");
  if (d.epi == EPI_SWIGLU_F16 && d.N % 8) throw Error(T0H_ERR_UNSUPPORTED, "gemm: SwiGLU hidden width must be a multiple of 8");
  if (d.row_add && (d.epi != EPI_STORE_F32 || !d.row_add_idx))
    throw Error(T0H_ERR_INVALID_ARG, "gemm: row_add needs EPI_STORE_F32 and an index array");
  if (d.a_f32) {
    if (d.epi != EPI_STORE_F32) throw Error(T0H_ERR_UNSUPPORTED, "gemm: f32 activations only with f32 stores");
    dispatch_type<true, EPI_STORE_F32>(d, force, s);
    return;
  }
  switch (d.epi) {
    case EPI_STORE_F32: dispatch_type<false, EPI_STORE_F32>(d, force, s); return;
    case EPI_STORE_F16: dispatch_type<false, EPI_STORE_F16>(d, force, s); return;
    case EPI_RESID_F32: dispatch_type<false, EPI_RESID_F32>(d, force, s); return;
    case EPI_SWIGLU_F16: dispatch_type<false, EPI_SWIGLU_F16>(d, force, s); return;
  }
  throw Error(T0H_ERR_INVALID_ARG, "gemm: unknown epilogue");
}

void launch_gemm(const GemmDesc& d, hipStream_t s) { launch_gemm_forced(d, 0, s); }

void launch_dequant(int type, const void* w, size_t n, float* out, hipStream_t s) {
  if (n == 0) return;
  if (!w || !out) throw Error(T0H_ERR_INVALID_ARG, "dequant: null pointer");
  const uint8_t* wb = static_cast<const uint8_t*>(w);
  switch (type) {
    case T0H_F32:
      hipLaunchKernelGGL(k_dequant<T0H_F32>, dim3((n + 255) / 256), dim3(256), 0, s, wb, n, out);
      break;
    case T0H_F16:
      hipLaunchKernelGGL(k_dequant<T0H_F16>, dim3((n + 255) / 256), dim3(256), 0, s, wb, n, out);
      break;
    case T0H_Q8_0:
    case T0H_Q4_0:
      if (n % 32) throw Error(T0H_ERR_SHAPE, "dequant: element count must be a multiple of 32");
      if (reinterpret_cast<uintptr_t>(w) % 2) throw Error(T0H_ERR_INVALID_ARG, "dequant: blocks must be 2-byte aligned");
      if (type == T0H_Q8_0)
        hipLaunchKernelGGL(k_dequant<T0H_Q8_0>, dim3((n / 32 + 255) / 256), dim3(256), 0, s, wb, n, out);
      else
        hipLaunchKernelGGL(k_dequant<T0H_Q4_0>, dim3((n / 32 + 255) / 256), dim3(256), 0, s, wb, n, out);
      break;
    default: throw Error(T0H_ERR_GGUF_TENSOR_TYPE, "dequant: unsupported type " + std::to_string(type));
  }
  check_hip(hipGetLastError(), "k_dequant launch");
}

}  // namespace t0h
